// moe_internal.h — types shared by the gfx950 kernels and the C ABI layer.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/moe_hip.h"

namespace moe {

constexpr int kBlk = 32;          // values per quantisation block
constexpr int kMaxExperts = 512;  // routed experts per layer the kernels support
constexpr int kMaxTopK = 64;      // experts per token the kernels support
constexpr int kMaxForced = 64;    // forced experts per layer

// Bytes of one 32-value block in format `dt` (F32 counts 32 floats).
__host__ __device__ inline int block_bytes(int dt) {
    switch (dt) {
    case MOE_DT_F32: return 128;
    case MOE_DT_Q8_0: return 34;
    case MOE_DT_Q4_0: return 18;
    case MOE_DT_Q5_0: return 22;
    default: return 0;
    }
}

// One weight matrix as the kernels see it: rows `stride` bytes apart.
struct MatDev {
    const uint8_t *ptr;
    uint32_t stride;  // bytes between rows (>= row bytes, multiple of 4)
    int32_t dt;
    int32_t rows;
    int32_t cols;
    // MFMA path: the block scales are multiplied by 2^wexp before the
    // weights are split into f16 pieces (exact: a power of two), so that the
    // matrix's largest |d q| lies in [2^14, 2^15).
    int32_t wexp;
    int32_t _pad = 0;
    // The matrix in the tiled layout of the one-subtile streaming kernel
    // (tile_matrix), or null.
    const uint8_t *tiled = nullptr;
};

// A SwiGLU expert: gate [I,H], up [I,H], down [H,I].  Routed experts occupy
// entries 0..E-1 of the layer's table; the shared expert, if any, entry E.
struct ExpertDev {
    MatDev m[3];
    int32_t inter;
    int32_t _pad;
};

// One-token experts: the work of one selected expert (or of the shared
// expert), as the dispatch kernel lays it out for the one-token kernels.
struct DecodeTask {
    const uint8_t *g, *u, *d;     // gate, up and down row 0
    float *h;                     // the expert's h row
    uint32_t gs, us, ds;          // row strides
    int32_t dcols;                // down width (I, or I_s for the shared expert)
    float w;                      // routing weight (shared expert: its sigmoid gate, or 1)
    int32_t live;                 // 0: slot not taken (fewer experts selected than k)
    int32_t _pad[2];
};

// Routing parameters the gating kernel needs.
struct GateParams {
    int32_t n_experts;
    int32_t top_k;          // effective k (after the routing override)
    int32_t sigmoid;
    int32_t norm_topk;
    int32_t n_group;
    int32_t topk_group;
    float routed_scale;
    float temp;             // > 0: logits /= temp
    int32_t n_forced;
    int32_t has_shared_gate;
    const float *e_bias;        // [E] or null
    // Interventions travel by value in the launch arguments, so a forward
    // already queued keeps the routing it was launched with.
    int32_t any_disabled;
    uint32_t disabled[kMaxExperts / 32];  // bit e: expert e may not be selected
    int32_t forced[kMaxForced];           // [n_forced]
};

// Per-call scratch, sized for max_t tokens (see moe_layer_reserve).
// K-half tiles of a launch's last round (tile_of): at most kTailPerXcd per
// XCD, one slot each.
constexpr int kTailPerXcd = 16;
constexpr int kTailSlots = 8 * kTailPerXcd;
// Bytes at the start of a workspace that must be zero before its first call
// (every call leaves them zero): the one-token route's block count and the
// K-half tiles' counts (at byte 256).
constexpr size_t kZeroBytes = 1024;

struct Workspace {
    int32_t max_t = 0;
    float *logits = nullptr;      // [T, E+1]
    int32_t *sel = nullptr;       // [T, k]
    float *wsel = nullptr;        // [T, k]
    float *shgate = nullptr;      // [T] sigmoid of the shared-expert gate
    int32_t *counts = nullptr;    // [E+1]
    int32_t *offsets = nullptr;   // [E+2]
    int32_t *perm_tok = nullptr;  // [T*k] token of each permuted row
    float *perm_w = nullptr;      // [T*k]
    int32_t *pos = nullptr;       // [T*k] permuted row of (t, slot)
    int32_t *hits = nullptr;      // [E+2] n, then experts ascending
    int32_t *tiles = nullptr;     // [4 * max_tiles] (group, m0, group's first tile, group's tiles) for the MFMA path
    DecodeTask *dtasks = nullptr; // [k + 1] one-token task table
    unsigned *route_count = nullptr;  // [1] finished router blocks (one-token route), zero between calls
    unsigned *tail_cnt = nullptr;     // [kTailSlots] K-half tiles' counts, zero between calls
    float *tail_part = nullptr;       // K-half tiles' partial sums (with tiled copies), or null
    int32_t *ntiles = nullptr;    // [1]
    int32_t *chunks = nullptr;    // [dispatch_chunks_upto(max_t) * E] per-chunk expert counts / first rows
    size_t chunks_cap = 0;        // entries of chunks
    uint16_t *xhi = nullptr, *xlo = nullptr;  // [T, H] f16 pieces of x (MFMA path)
    int32_t *xex = nullptr;       // [T] their row exponents
    uint16_t *hhi = nullptr, *hlo = nullptr;  // [T*k, I] f16 pieces of h (MFMA path)
    int32_t *hex = nullptr;       // [T*k]
    uint16_t *hshi = nullptr, *hslo = nullptr;  // [T, I_s] pieces of hs
    int32_t *hsex = nullptr;      // [T]
    uint8_t *xq = nullptr;        // [batch_t, H/64] activation units (few-tokens path)
    uint8_t *hq = nullptr;        // [batch_t * k, I/64] units of h
    uint8_t *hsq = nullptr;       // [batch_t, I_s/64] units of hs
    uint8_t *dq = nullptr;        // [k + 1, max(I, I_s)/64] units of the one-token path's h rows
    int batch_t = 0;              // tokens the unit buffers have room for
    float *h = nullptr;           // [T*k, I] routed SwiGLU activations (f32)
    float *hs = nullptr;          // [T, I_s] shared-expert activations
    float *y = nullptr;           // [parts][T*k, H] routed expert outputs (parts: split K of the down projection)
    float *ys = nullptr;          // [parts][T, H] shared-expert outputs
    size_t y_rows = 0, ys_rows = 0;  // rows y and ys have room for
    unsigned long long *stats = nullptr;  // [4] fallback when the caller passes none
    void *base = nullptr;         // single allocation backing all of the above
    size_t bytes = 0;
};

// --------------------------------------------------------------- launchers
// Each returns hipSuccess or the launch error.

// Router logits, bit-exact to the reference's dot (src/quant.rs:386-420):
// logits[t][e] = W[e] . x[t] for e < n_rows, divided by temp (e < E only)
// when temp > 0.  Row E (if n_rows == E+1) is the shared-expert gate.
hipError_t launch_router(const float *W, const float *x, int T, int n_rows, int E, int H, float temp, float *logits,
                         hipStream_t s);

// Gating + top-k + weights per token (src/model.rs:855-897).
hipError_t launch_gating(const float *logits, int ld, int T, const GateParams &p, int32_t *sel, float *wsel,
                         float *shgate, unsigned long long *stats, hipStream_t s);

// Stable token->expert dispatch (src/model.rs:900-930) plus the work lists.
struct DispatchArgs {
    const int32_t *sel;
    const float *wsel;
    int T, k, E;
    int has_shared;
    int bm;                       // MFMA M-tile (0: no tile list)
    const unsigned long long *expert_bytes;  // [E]
    const uint32_t *prev;         // [E+1] or null
    int32_t *counts, *offsets, *perm_tok, *pos, *hits, *tiles, *ntiles;
    float *perm_w;
    moe_route *routes;            // [T, k] or null
    uint32_t *hits_out;           // [E+1] or null
    unsigned long long *stats;    // [4]
    float *shgate_out;            // [T] gating output (one-token route kernel)
    // One token (T = 1) on the one-token kernels: their task table.
    DecodeTask *dtasks;           // [dk_bound + has_shared] or null
    const ExpertDev *experts;     // device table [E+1]
    float *h, *hs;                // h rows the tasks point at
    const float *shgate;          // [1] or null
    int I, dk_bound;
};
// More than 512 tokens: three launches (count per
// chunk, scan, place per chunk) using chunk_scratch [dispatch_chunks(T) * E]
// ints (chunk_cap of them: a launch that would need more fails with
// hipErrorInvalidValue); otherwise one block.  The permuted rows are the
// same either way.
int dispatch_chunks(int T);
// The most chunks any T' <= T takes: dispatch_chunks is not monotonic (its
// chunks widen past 4096 tokens), so scratch for up to T tokens holds this.
int dispatch_chunks_upto(int T);
hipError_t launch_dispatch(const DispatchArgs &a, int32_t *chunk_scratch, size_t chunk_cap, hipStream_t s);

// Router + gating + dispatch of one token in one launch (n_rows blocks; the
// last to finish gates and dispatches).  `counter` is zero between calls.
bool route_one_ok(int H, int E);
hipError_t launch_route_one(const float *W, const float *x, int n_rows, int E, int H, float temp, float *logits,
                            const GateParams &p, const DispatchArgs &d, unsigned *counter, hipStream_t s);

// y = the gates' exp (glibc expf port) over n values; diagnostics.
hipError_t launch_expf(const float *x, float *y, size_t n, hipStream_t s);

// Decode-path expert GEMVs (fp32, weights dequantised exactly in registers).
struct GemvArgs {
    const ExpertDev *experts;     // device table [E+1]
    const int32_t *hits;          // [E+2]
    const int32_t *counts, *offsets, *perm_tok;
    const float *perm_w;          // [T*k] routing weight of each permuted row
    const float *shgate;          // [T] sigmoid shared-expert gate, or null
    const float *x;               // [T, H]
    float *h, *hs;                // routed [T*k, I], shared [T, I_s]
    float *y, *ys;                // routed [T*k, H], shared [T, H]
    float *out, *residual;        // fused combine: [T, H] (residual may be null)
    int T, H, I, I_s, E;
    int task_bound;               // routed tasks launched (>= hits[0])
    int has_shared;
};
hipError_t launch_gemv_up(const GemvArgs &a, const ExpertDev &host_e0, const ExpertDev *host_shared, hipStream_t s);
hipError_t launch_gemv_down(const GemvArgs &a, const ExpertDev &host_e0, const ExpertDev *host_shared, hipStream_t s);
// The down projection of table entry a.E alone (a.task_bound == 0): the
// plain projection ys = W hs over all a.T tokens.
hipError_t launch_gemv_down_single(const GemvArgs &a, const ExpertDev &ex, hipStream_t s);
// dst[i] += src[i] for n values.
hipError_t launch_add(float *dst, const float *src, size_t n, hipStream_t s);
// y[i] = parts[i] + parts[n + i] + ... (k parts, in order); residual[i] +=
// y[i] when residual is not null.
hipError_t launch_sum_parts(const float *parts, int k, size_t n, float *y, float *residual, hipStream_t s);
// Down projection with the combine, shared expert and residual folded in
// (T <= kFusedMaxT): writes out (and residual) directly.
constexpr int kFusedMaxT = 8;
hipError_t launch_gemv_down_combine(const GemvArgs &a, const ExpertDev &host_e0, const ExpertDev *host_shared,
                                    hipStream_t s);

// Exact-order expert GEMVs (bit-identical to the reference's dot).
hipError_t launch_gemv_exact(bool up, const GemvArgs &a, hipStream_t s);

// One-token experts on integer dot products (three-level int8 activations).
struct DecodeArgs {
    const DecodeTask *tasks;      // [k_bound + n_shared], written by the dispatch kernel
    const int32_t *hits;          // [E+2]
    float *h, *hs;                // h: routed [k, I], shared [I_s]
    int has_gate;                 // the shared expert has a sigmoid gate
    float *y, *ys;                // routed [k, H], shared [H]
    float *out, *residual;        // [H] (residual may be null)
    int H, I, I_s, E;
    int k_bound;                  // routed tasks launched (>= hits[0])
    int n_shared;                 // 1 if the shared expert is part of the launch
    uint8_t *hq;                  // activation units of h: task t's unit u at (t * hq_units + u) * kQUnitBytes
    int hq_units;                 // unit slots per task (max(I, I_s) / 64)
    const float *addend;          // [H] added to out after the routed sum (the shared expert's gated output
                                  // when it needs a down launch of its own), or null
};
// Whether the one-token kernels take these widths and formats, and whether
// a down-projection block holds k routed experts (and the shared one).
constexpr int kDecodeMaxWaves = 16;  // waves of a down-projection block
bool decode_supported(int H, int I, int I_s, int dt_routed, int dt_shared);
bool decode_fits(int I, int I_s, int k, int has_shared, int dt_routed, int dt_shared);
// `encoded`: the launch also encoded h into a.hq (the unit-aligned kernel),
// so launch_decode_encode is not needed.
hipError_t launch_decode_up(const DecodeArgs &a, const float *x, int dt_routed, int dt_shared, bool &encoded,
                            hipStream_t s);
// Every live task's h (f32) to activation units at a.hq, one wavefront per unit.
hipError_t launch_decode_encode(const DecodeArgs &a, hipStream_t s);
// The one-token gate/up kernel choice (moe_debug_decode_kernel); returns
// the previous one.
int set_decode_kernel(int choice);
// The MFMA kernels (moe_debug_mfma_kernel): 0 two-pass, 1 three-pass;
// returns the previous one.
int set_mfma_kernel(int choice);
// The down projection and combine over the units of h.
hipError_t launch_decode_down(const DecodeArgs &a, int dt_routed, int dt_shared, hipStream_t s);
// Whether the shared expert's down projection runs as a launch of its own
// (its format, or its units per lane, differ from the routed experts').
bool decode_shared_apart(int I, int I_s, int dt_routed, int dt_shared);

// Prefill-path grouped GEMMs on MFMA in f32 precision: activations and the
// dequantised weights are each split into two f16 pieces (hi + lo, exact for
// d q; 22 significant bits for activations, with a per-row power-of-two scale
// keeping both pieces in f16's normal range), and hi.hi + hi.lo + lo.hi are
// accumulated in f32 by V_MFMA_F32_32X32X16_F16.
struct MfmaArgs {
    const ExpertDev *experts;
    const int32_t *tiles, *ntiles;
    const int32_t *counts, *offsets, *perm_tok;
    const uint16_t *xhi, *xlo;    // [T, H] f16 pieces of x * 2^xex[row]
    const int32_t *xex;           // [T]
    float *h, *hs;                // f32 [T*k, I], [T, I_s] (gate/up output)
    const uint16_t *hhi, *hlo;    // [T*k, I] pieces of h (down input)
    const int32_t *hex;           // [T*k]
    const uint16_t *hshi, *hslo;  // [T, I_s] pieces of hs
    const int32_t *hsex;          // [T]
    float *y, *ys;                // f32 [T*k, H], [T, H]
    size_t ypart, yspart;         // elements between the K parts of y, ys
    int T, H, I, I_s, E;
    int k = 1;                    // experts per token (routed launches)
    int max_tiles;                // grid width of the routed launch: >= the routed tiles
    int shared_tiles;             // tiles of the shared expert at the end of the tile list (0 if none)
    int ksplit;                   // down projection: K parts (1, 2 or 4), part p written at y + p * ypart
    int xcd_cus;                  // CUs per XCD (set by the launchers)
    // One-subtile gate/up tiles split along K in a launch's last round:
    // partial sums [slots][2][8 waves][16][64] f32 and a count per slot
    // (zero between calls), or null (no such split).
    float *tail_part = nullptr;
    unsigned *tail_cnt = nullptr;
};
// Token tile of the MFMA kernels for a layer whose matrices have formats
// dts[0..n): 160, or 128 when a Q8_0 matrix leaves LDS room for fewer rows.
int mfma_tile_m(const int *dts, int n);
// The token tile of one routed call of t tokens, k experts each, of E.
int mfma_call_tile(int layer_bm, int t, int k, int E);
bool mfma_format_ok(int dt);
bool mfma_fits(size_t t, size_t k, size_t H, size_t I, size_t I_s);
constexpr int kMaxKSplit = 4;
int mfma_down_ksplit(int m_tiles, int n_rows, int K, int K_shared);
// up: gate/up + SwiGLU; down: down projection.  Routed tiles come from the
// dispatch list built with tile `bm`; the shared expert (sh != null) gets its
// own launch.
hipError_t launch_mfma(bool up, const MfmaArgs &a, int bm, const ExpertDev &e0, const ExpertDev *sh, hipStream_t s);
// One matrix over all T tokens (the shared-expert tiles alone): the plain
// projection y = W x on the matrix cores.  The matrix is table entry
// a.E (a.experts[a.E]); the activations are the shared expert's pieces
// (hshi, hslo, hsex for the down form) and the output goes to ys.
hipError_t launch_mfma_single(bool up, const MfmaArgs &a, int bm, const ExpertDev &ex, hipStream_t s);
// Rows [rows, cols] of f32 into f16 pieces: hi + lo = v * 2^ex[row] to
// 22 bits, ex chosen per row so that its largest |v| scales into
// [2^14, 2^15) (0 for an all-zero or non-finite row).  cols % 4 == 0.
hipError_t launch_split_rows(const float *src, int rows, int cols, uint16_t *hi, uint16_t *lo, int32_t *ex,
                             hipStream_t s);

// The streaming expert kernels (expert_stream.hip): eight waves per tile of
// bm = 32, 64, 128 or 160 tokens (160 only for Q4_0 / Q5_0) x 256 weight
// rows, the same arguments and activation pieces as launch_mfma.  With
// every matrix of the launch tiled (MatDev::tiled), 32-token tiles stream
// their weights through registers from the tiled copy.
int stream_tile(double tokens, bool q8);
// The tile of a launch whose one tile holds exactly `tokens` (the shared
// expert): 32 up to 32 tokens, else stream_tile's.
int stream_tile_exact(int tokens, bool q8);
// The tiled layout: bytes of matrix m's copy (0 if its format or shape has
// none: Q4_0 / Q5_0 / Q8_0 with cols % 64 == 0), and the copy written to
// dst (tiled_bytes(m) bytes of device memory) on stream s.
size_t tiled_bytes(const MatDev &m);
hipError_t tile_matrix(const MatDev &m, uint8_t *dst, hipStream_t s);
hipError_t launch_stream(bool up, const MfmaArgs &a, int bm, const ExpertDev &e0, const ExpertDev *sh, hipStream_t s);
hipError_t launch_stream_single(bool up, const MfmaArgs &a, int bm, const ExpertDev &ex, hipStream_t s);
// Largest |d| (f16 bits) of every block scale of matrix m of expert g into
// out[3 g + m], for the n experts of the table (F32 matrices give 0).
hipError_t launch_scale_max(const ExpertDev *experts, int n, unsigned *out, hipStream_t s);

// Weighted combine in ascending expert order + shared expert + residual
// (src/model.rs:936-942, 956-970, 680-683).
// Few tokens per expert: the experts' rows dotted with int8-encoded
// activations (qact.h), NT tokens per tile, every weight unit loaded once
// per tile.  Tiles come from the dispatch tile list built with bm = NT.
struct BatchArgs {
    const ExpertDev *experts;
    const int32_t *tiles, *ntiles;
    const int32_t *counts, *offsets, *perm_tok;
    const uint8_t *xq;            // [T, H/64] activation units
    float *h, *hs;                // f32 [T*k, I], [T, I_s]
    const uint8_t *hq, *hsq;      // [T*k, I/64], [T, I_s/64] units of h, hs
    float *y, *ys;                // f32 [parts][T*k, H], [parts][T, H]
    size_t ypart, yspart;         // elements between the K parts of y, ys
    int T, H, I, I_s, E;
    int max_tiles;                // grid height of the routed launch: >= the routed tiles
    int shared_tiles;             // tiles of the shared expert at the end of the tile list (0 if none)
    int ksplit;                   // down projection: K parts, part p written at y + p * ypart
    int nt;                       // tokens per tile (the dispatch's bm): 1 or 2
};
constexpr int kBatchMaxT = 256;   // largest t the few-tokens path is sized for
// Formats and widths the few-tokens kernels take.
bool batch_supported(int H, int I, int I_s, int dt_routed, int dt_shared);
// Tokens per tile (the dispatch's bm) for hidden width H and t tokens with
// k experts each over E experts: 1 for rows wider than 4096 or at most one
// token per expert on average, else 2.
int batch_tile_tokens(int H, int t, int k, int E);
// K parts of the down projection (each part at most 64 units per row).
int batch_ksplit(int I, int I_s);
// Rows [rows, cols] of f32 (cols a multiple of 64) to activation units.
hipError_t launch_qenc(const float *src, int rows, int cols, uint8_t *dst, hipStream_t s);
hipError_t launch_batch_up(const BatchArgs &a, const ExpertDev &e0, const ExpertDev *sh, hipStream_t s);
hipError_t launch_batch_down(const BatchArgs &a, const ExpertDev &e0, const ExpertDev *sh, hipStream_t s);
// The shared expert's tiles alone (what the two launchers above add for sh).
hipError_t launch_batch_up_shared(const BatchArgs &a, const ExpertDev &sh, hipStream_t s);
hipError_t launch_batch_down_shared(const BatchArgs &a, const ExpertDev &sh, hipStream_t s);

struct CombineArgs {
    const float *y, *ys;
    int parts;                    // K parts of y and ys, summed in order before weighting
    size_t ypart, yspart;         // elements between parts
    const int32_t *pos;
    const int32_t *sel;
    const float *wsel;
    const float *shgate;          // [T] or null
    float *out, *residual;
    int T, H, k, has_shared;
};
hipError_t launch_combine(const CombineArgs &a, hipStream_t s);

}  // namespace moe
