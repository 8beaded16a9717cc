// moe_abi.hip — the C ABI of libmoe_hip: contexts, uploaded regions, layers
// and the forward orchestration (router -> gating -> dispatch -> experts ->
// combine), all asynchronous on the caller's stream.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <memory>
#include <mutex>
#include <string>
#include <vector>

#include "moe_internal.h"
#include "qact.h"

using namespace moe;


namespace moe {

thread_local std::string g_err;

// Records the message moe_last_error returns (the host-only sources report
// through it too) and passes the status code through.
int fail(int code, const char *fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_err = buf;
    return code;
}

}  // namespace moe


namespace {

int hip_fail(hipError_t e, const char *what) { return fail(MOE_EHIP, "%s: %s", what, hipGetErrorString(e)); }

struct DeviceGuard {
    int prev = -1;
    explicit DeviceGuard(int dev) {
        hipGetDevice(&prev);
        if (prev != dev) hipSetDevice(dev);
    }
    ~DeviceGuard() {
        int cur = -1;
        hipGetDevice(&cur);
        if (prev >= 0 && cur != prev) hipSetDevice(prev);
    }
};

struct Region {
    void *ptr = nullptr;
    uint64_t bytes = 0;
};

// Forward path for a call.
enum Path { kExact = 1, kGemv = 2, kMfma = 3, kDecode = 4, kBatch = 5, kStream = 6 };

// A normal or subnormal f16 magnitude (bits & 0x7fff, below inf) as float.
float f16_bits_to_float(unsigned bits) {
    const int e = (int)(bits >> 10) & 31, m = (int)(bits & 1023);
    return e == 0 ? std::ldexp((float)m, -24) : std::ldexp((float)(1024 + m), e - 25);
}

// A workspace a layer owns for one stream (moe_layer_forward).
struct StreamWs {
    hipStream_t stream;
    Workspace w;
    int k;
};
// An outgrown or released workspace: free once `done` (recorded on its
// stream when it was retired, after the last work that used it) has
// completed; without an event, at moe_layer_destroy.
struct Retired {
    void *base;
    hipEvent_t done;
};

}  // namespace

struct moe_ctx {
    int device = 0;
    std::mutex mu;
    std::vector<Region> regions;
    // The stream that runs the encoding of x beside the routing and the
    // shared expert's kernels beside the routed ones (few-tokens and MFMA
    // paths), and the events that fork it from the caller's stream, mark the
    // end of x's encoding, and join it back; side_mu makes each
    // record-and-wait pair atomic between callers.  Null if they could not
    // be created.
    hipStream_t side = nullptr;
    hipEvent_t ev_fork = nullptr, ev_join = nullptr, ev_x = nullptr;
    std::mutex side_mu;
};

struct moe_layer {
    moe_ctx *ctx = nullptr;
    int H = 0, E = 0, I = 0, I_s = 0;
    int top_k_spec = 0;
    int gate = 0, norm_topk = 1, n_group = 1, topk_group = 1;
    float routed_scale = 1.0f;
    bool has_shared = false, has_shared_gate = false;
    bool fast_ok = false, mfma_ok = false, decode_ok = false, batch_ok = false;
    int mfma_bm = 160;  // token tile of the MFMA kernels for this layer's formats
    // device memory owned by the layer
    float *router = nullptr;             // [E + has_shared_gate, H]
    const float *e_bias = nullptr;       // points into a region
    ExpertDev *experts_dev = nullptr;    // [E + 1]
    unsigned long long *expert_bytes = nullptr;  // [E]
    std::vector<ExpertDev> experts_host;
    // Everything below may change between calls; `mu` guards it.  A call
    // takes a snapshot of the routing and the mode under the lock.
    std::mutex mu;
    int mode = 0;  // 0 auto, else a Path
    float temp = 0.0f;
    int top_k_override = 0;
    int n_forced = 0;
    int32_t forced[kMaxForced] = {};
    uint32_t disabled[kMaxExperts / 32] = {};
    bool any_disabled = false;
    std::vector<StreamWs> ws;            // one workspace per stream used with moe_layer_forward
    std::vector<Retired> retired;        // outgrown or released workspaces, not yet freed
    void *tiled_mem = nullptr;           // the experts' tiled copies (moe_layer_set_tiled), one allocation
    int reserved_t = 0, reserved_k = 0;  // after moe_layer_reserve: calls beyond these fail
    // stage timing
    bool profile = false;
    struct StageRec {
        int stage;
        hipEvent_t a, b;
    };
    std::vector<hipEvent_t> event_pool;
    std::vector<StageRec> pending;
    double stage_ms[MOE_STAGES] = {};
    uint64_t stage_n[MOE_STAGES] = {};
};

namespace {

hipEvent_t take_event(moe_layer *L) {
    if (!L->event_pool.empty()) {
        hipEvent_t e = L->event_pool.back();
        L->event_pool.pop_back();
        return e;
    }
    hipEvent_t e = nullptr;
    hipEventCreate(&e);
    return e;
}

// Runs `fn` (which launches one stage's kernels on `s`) between two events
// when profiling is on.
template <class F>
int stage(moe_layer *L, bool profile, int id, hipStream_t s, F fn) {
    if (!profile) return fn();
    hipEvent_t a, b;
    {
        std::lock_guard<std::mutex> g(L->mu);
        a = take_event(L), b = take_event(L);
    }
    hipEventRecord(a, s);
    const int rc = fn();
    hipEventRecord(b, s);
    std::lock_guard<std::mutex> g(L->mu);
    L->pending.push_back({id, a, b});
    return rc;
}

const Region *region_of(moe_ctx *ctx, uint64_t id) {
    if (id >= ctx->regions.size() || !ctx->regions[id].ptr) return nullptr;
    return &ctx->regions[id];
}

bool dt_ok(int dt) { return dt == MOE_DT_F32 || dt == MOE_DT_Q4_0 || dt == MOE_DT_Q5_0 || dt == MOE_DT_Q8_0; }

// Resolve a view to a device matrix, checking format, shape and bounds
// (Rec::fits_in, src/store.rs:44-46).
int resolve(moe_ctx *ctx, const moe_tensor &t, int rows, int cols, const char *what, MatDev &out) {
    if (!dt_ok(t.dt)) return fail(MOE_EUNSUP, "%s: storage format %d is not supported (F32, Q4_0, Q5_0, Q8_0)", what, t.dt);
    if (t.rows != rows || t.cols != cols)
        return fail(MOE_EINVAL, "%s: shape [%d, %d], expected [%d, %d]", what, t.rows, t.cols, rows, cols);
    if (t.dt != MOE_DT_F32 && cols % kBlk != 0)
        return fail(MOE_EINVAL, "%s: %d columns is not a whole number of 32-value blocks", what, cols);
    const Region *r = region_of(ctx, t.region);
    if (!r) return fail(MOE_EINVAL, "%s: unknown region %llu", what, (unsigned long long)t.region);
    const uint64_t rb = moe_row_bytes(t.dt, (uint64_t)cols);
    const uint64_t len = rb * (uint64_t)rows;
    if (t.offset > r->bytes || len > r->bytes - t.offset)
        return fail(MOE_EINVAL, "%s: %llu bytes at offset %llu overrun its %llu-byte region", what,
                    (unsigned long long)len, (unsigned long long)t.offset, (unsigned long long)r->bytes);
    out.ptr = static_cast<const uint8_t *>(r->ptr) + t.offset;
    out.stride = (uint32_t)rb;
    out.dt = t.dt;
    out.rows = rows;
    out.cols = cols;
    return MOE_OK;
}

bool present(const moe_tensor &t) { return t.dt >= 0; }

// A matrix can take the fast kernels: 4-byte aligned rows of whole 64-value
// units, at most 256 units wide.
bool fast_mat(const MatDev &m) {
    return ((uintptr_t)m.ptr % 4 == 0) && (m.stride % 4 == 0) && (m.cols % 64 == 0) && (m.cols / 64 <= 256);
}


int effective_k_locked(const moe_layer *L) {
    int k = L->top_k_override > 0 ? L->top_k_override : L->top_k_spec;
    return std::min(k, L->E);
}

size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

// Whether the few-tokens kernels beat MFMA tiles.  Their cost is the
// weight bytes of every tile (an expert's weights are read once per tile of
// nt tokens).  Measured on MI355X against the two-pass MFMA kernels (ms per
// layer, few-tokens against MFMA): with two-token tiles and rows of 2048
// they win while the hit experts average at most 4 tokens (Qwen3 T=64 0.277
// against 0.293; V2-Lite T=64 at 6 tokens loses, 0.405 against 0.311), with
// rows of 4096 at most 3 (Mixtral T=8 at 2 tokens 0.275 against 0.391, T=16
// at 4 loses, 0.457 against 0.412), with one-token tiles (rows wider than
// 4096) at most 1.5 (DeepSeek-V3 T=32 at 1 token 1.054 against 1.116).
bool batch_pays(int t, int k, int E, int H, int nt) {
    if (t < 2 || t > kBatchMaxT) return false;
    const long long rows = (long long)t * k, hit = std::min<long long>(E, rows);
    if (nt < 2) return 2 * rows <= 3 * hit;
    return rows <= (H >= 4096 ? 3 : 4) * hit;
}

// Byte layout of a workspace for up to max_t tokens of k experts each.
// The first 256 bytes hold the counters that must be zero between calls
// (they sit at the same place whatever max_t is); every array starts on a
// 256-byte boundary.  Assigns w's pointers when base is given; returns the
// total size.
size_t ws_layout(const moe_layer *L, int max_t, int k, Workspace *w, char *base) {
    const size_t T = (size_t)max_t, E = (size_t)L->E, H = (size_t)L->H;
    const size_t I = (size_t)std::max(L->I, 1), Is = (size_t)std::max(L->I_s, 1);
    // Tiles of one token or more (the few-tokens path), or bm (MFMA).
    const size_t max_tiles = T * k + E + 2 + T;
    // Activation units for the few-tokens path, which runs up to kBatchMaxT tokens.
    const size_t Tb = L->batch_ok ? std::min<size_t>(T, kBatchMaxT) : 0;
    // f16 pieces of the MFMA path.
    const size_t Tm = L->mfma_ok ? T : 0;
    // Room for the K parts of a split MFMA / few-tokens down projection.
    // Splitting only pays for small grids, so parts after the first are
    // bounded in rows.
    const size_t extra = (L->mfma_ok || L->batch_ok) ? (kMaxKSplit - 1) * std::min<size_t>(T * k, 8192) : 0;
    const size_t y_rows = T * k + extra, ys_rows = T + extra;
    Workspace tmp;
    Workspace &x = w ? *w : tmp;
    x = Workspace();
    x.max_t = max_t;
    x.batch_t = (int)Tb;
    x.y_rows = y_rows;
    x.ys_rows = ys_rows;
    struct Item {
        void **dst;
        size_t bytes;
    };
    const Item items[] = {
        {(void **)&x.route_count, kZeroBytes},  // with the K-half tiles' counts
        {(void **)&x.tail_part, L->tiled_mem ? (size_t)kTailSlots * 2 * 8 * 16 * 64 * 4 : 0},
        {(void **)&x.logits, T * (E + 1) * 4},
        {(void **)&x.sel, T * k * 4},
        {(void **)&x.wsel, T * k * 4},
        {(void **)&x.shgate, T * 4},
        {(void **)&x.counts, (E + 2) * 4},
        {(void **)&x.offsets, (E + 2) * 4},
        {(void **)&x.perm_tok, T * k * 4},
        {(void **)&x.perm_w, T * k * 4},
        {(void **)&x.pos, T * k * 4},
        {(void **)&x.hits, (E + 2) * 4},
        {(void **)&x.tiles, 4 * max_tiles * 4},
        {(void **)&x.dtasks, (size_t)(k + 1) * sizeof(DecodeTask)},
        {(void **)&x.ntiles, 4},
        {(void **)&x.chunks, (size_t)dispatch_chunks_upto((int)T) * E * 4},
        {(void **)&x.xhi, Tm * H * 2},
        {(void **)&x.xlo, Tm * H * 2},
        {(void **)&x.xex, Tm * 4},
        {(void **)&x.hhi, Tm * k * I * 2},
        {(void **)&x.hlo, Tm * k * I * 2},
        {(void **)&x.hex, Tm * k * 4},
        {(void **)&x.hshi, L->has_shared ? Tm * Is * 2 : 0},
        {(void **)&x.hslo, L->has_shared ? Tm * Is * 2 : 0},
        {(void **)&x.hsex, L->has_shared ? Tm * 4 : 0},
        {(void **)&x.xq, Tb * (H / 64) * kQUnitBytes},
        {(void **)&x.hq, Tb * k * (I / 64) * kQUnitBytes},
        {(void **)&x.hsq, Tb * (Is / 64) * kQUnitBytes},
        {(void **)&x.dq, L->decode_ok ? (size_t)(k + 1) * (std::max(I, Is) / 64) * kQUnitBytes : 0},
        {(void **)&x.h, T * k * I * 4},
        {(void **)&x.hs, T * Is * 4},
        {(void **)&x.y, y_rows * H * 4},
        {(void **)&x.ys, ys_rows * H * 4},
        {(void **)&x.stats, 4 * 8},
    };
    size_t off = 0;
    for (const Item &it : items) {
        if (base) *it.dst = base + off;
        off += align_up(std::max<size_t>(it.bytes, 1), 256);
    }
    x.base = base;
    x.bytes = off;
    x.chunks_cap = (size_t)dispatch_chunks_upto((int)T) * E;
    if (base) x.tail_cnt = x.route_count + 64;
    if (!L->tiled_mem) x.tail_part = nullptr;
    return off;
}

// Retire a stream's workspace: queued work may still use it, so it is
// freed only once an event recorded on the stream now has completed.
void retire_ws(moe_layer *L, void *base, hipStream_t s) {
    hipEvent_t ev = nullptr;
    if (hipEventCreateWithFlags(&ev, hipEventDisableTiming) == hipSuccess && hipEventRecord(ev, s) != hipSuccess) {
        hipEventDestroy(ev);
        ev = nullptr;
    }
    L->retired.push_back({base, ev});
}
// Free the retired workspaces whose event has completed (a query, no wait).
void reap_ws(moe_layer *L) {
    for (size_t i = 0; i < L->retired.size();) {
        Retired &r = L->retired[i];
        if (r.done && hipEventQuery(r.done) == hipSuccess) {
            hipFree(r.base);
            hipEventDestroy(r.done);
            r = L->retired.back();
            L->retired.pop_back();
        } else {
            i++;
        }
    }
}

// The workspace of `stream` for t tokens (moe_layer_forward): the layer
// keeps one per stream, so calls on different streams never share scratch.
// Grows without waiting for the device, geometrically (at least 1.5 times
// the old size, in 64-token steps) so that rising token counts allocate
// O(final size) in total; the outgrown workspace is retired and freed at a
// later growth once the work queued on it has finished.  A reserved layer
// does not grow: a larger call fails.
int stream_ws(moe_layer *L, hipStream_t s, int t, int k, Workspace &out) {
    std::lock_guard<std::mutex> g(L->mu);
    StreamWs *cur = nullptr;
    for (StreamWs &e : L->ws)
        if (e.stream == s) cur = &e;
    if (cur && t <= cur->w.max_t && k <= cur->k) {
        out = cur->w;
        return MOE_OK;
    }
    if (L->reserved_t > 0 && (t > L->reserved_t || k > L->reserved_k))
        return fail(MOE_EINVAL, "%d tokens of %d experts exceed the reservation of %d tokens of %d experts", t, k,
                    L->reserved_t, L->reserved_k);
    int max_t = std::max(t, L->reserved_t), kk = std::max(k, L->reserved_k);
    if (cur) {
        if (t > cur->w.max_t && L->reserved_t == 0) {
            const long long grown = (long long)cur->w.max_t + cur->w.max_t / 2;
            max_t = (int)std::max<long long>(t, std::min<long long>((grown + 63) / 64 * 64, 1 << 24));
        }
        max_t = std::max(max_t, cur->w.max_t), kk = std::max(kk, cur->k);
    }
    reap_ws(L);
    const size_t bytes = ws_layout(L, max_t, kk, nullptr, nullptr);
    void *base = nullptr;
    hipError_t e = hipMalloc(&base, bytes);
    if (e != hipSuccess) return fail(MOE_ENOMEM, "workspace of %zu bytes for %d tokens: %s", bytes, max_t, hipGetErrorString(e));
    if ((e = hipMemset(base, 0, kZeroBytes)) != hipSuccess) {
        hipFree(base);
        return fail(MOE_EHIP, "workspace counters: %s", hipGetErrorString(e));
    }
    Workspace w;
    ws_layout(L, max_t, kk, &w, static_cast<char *>(base));
    if (cur) {
        retire_ws(L, cur->w.base, s);
        cur->w = w;
        cur->k = kk;
    } else {
        L->ws.push_back({s, w, kk});
    }
    out = w;
    return MOE_OK;
}

// What a call reads of the layer's mutable state, taken under the lock.
struct CallState {
    int mode;
    int k;
    bool profile;
    bool side = true;  // the shared expert may run on the context's side stream
    GateParams gp;
};

CallState snapshot(moe_layer *L) {
    std::lock_guard<std::mutex> g(L->mu);
    CallState c;
    c.mode = L->mode;
    c.k = effective_k_locked(L);
    c.profile = L->profile;
    GateParams &p = c.gp;
    p = GateParams{};
    p.n_experts = L->E;
    p.top_k = c.k;
    p.sigmoid = L->gate == MOE_GATE_SIGMOID;
    p.norm_topk = L->norm_topk;
    p.n_group = L->n_group;
    p.topk_group = L->topk_group;
    p.routed_scale = L->routed_scale;
    p.temp = L->temp;
    p.n_forced = L->n_forced;
    p.has_shared_gate = L->has_shared_gate;
    p.e_bias = L->e_bias;
    p.any_disabled = L->any_disabled;
    std::memcpy(p.disabled, L->disabled, sizeof p.disabled);
    std::memcpy(p.forced, L->forced, sizeof p.forced);
    return c;
}

// Router, gating and dispatch; shared by forward and route.
int route_and_dispatch(moe_layer *L, const CallState &c, Workspace &w, const float *x, int t, int bm, bool decode,
                       moe_route *routes, uint32_t *hits, const uint32_t *prev, uint64_t *stats, float *logits_out,
                       hipStream_t s) {
    const int k = c.k;
    const int n_rows = L->E + (L->has_shared_gate ? 1 : 0);
    hipError_t e = hipSuccess;
    unsigned long long *st = stats ? reinterpret_cast<unsigned long long *>(stats) : w.stats;
    const GateParams &p = c.gp;
    DispatchArgs a{};
    a.sel = w.sel;
    a.wsel = w.wsel;
    a.T = t;
    a.k = k;
    a.E = L->E;
    a.has_shared = L->has_shared;
    a.bm = bm;
    a.expert_bytes = L->expert_bytes;
    a.prev = prev;
    a.counts = w.counts;
    a.offsets = w.offsets;
    a.perm_tok = w.perm_tok;
    a.pos = w.pos;
    a.hits = w.hits;
    a.tiles = w.tiles;
    a.ntiles = w.ntiles;
    a.perm_w = w.perm_w;
    a.routes = routes;
    a.hits_out = hits;
    a.stats = st;
    a.shgate_out = w.shgate;
    if (decode) {
        a.dtasks = w.dtasks;
        a.experts = L->experts_dev;
        a.h = w.h;
        a.hs = w.hs;
        a.shgate = L->has_shared_gate ? w.shgate : nullptr;
        a.I = L->I;
        a.dk_bound = k;
    }
    auto copy_logits = [&]() -> int {
        if (!logits_out) return MOE_OK;
        if ((e = hipMemcpy2DAsync(logits_out, (size_t)L->E * 4, w.logits, (size_t)n_rows * 4, (size_t)L->E * 4, t,
                                  hipMemcpyDeviceToDevice, s)) != hipSuccess)
            return hip_fail(e, "logits copy");
        return MOE_OK;
    };
    if (t == 1 && route_one_ok(L->H, L->E)) {
        // One token: router, gating and dispatch in a single launch.
        int rc = stage(L, c.profile, 0, s, [&] {
            e = launch_route_one(L->router, x, n_rows, L->E, L->H, p.temp, w.logits, p, a, w.route_count, s);
            return e == hipSuccess ? MOE_OK : hip_fail(e, "one-token route kernel");
        });
        return rc ? rc : copy_logits();
    }
    int rc = stage(L, c.profile, 0, s, [&] {
        e = launch_router(L->router, x, t, n_rows, L->E, L->H, p.temp, w.logits, s);
        return e == hipSuccess ? MOE_OK : hip_fail(e, "router kernel");
    });
    if (rc) return rc;
    rc = stage(L, c.profile, 1, s, [&] {
        e = launch_gating(w.logits, n_rows, t, p, w.sel, w.wsel, w.shgate, st, s);
        return e == hipSuccess ? MOE_OK : hip_fail(e, "gating kernel");
    });
    if (rc) return rc;
    if ((rc = copy_logits())) return rc;
    return stage(L, c.profile, 2, s, [&] {
        e = launch_dispatch(a, w.chunks, w.chunks_cap, s);
        return e == hipSuccess ? MOE_OK : hip_fail(e, "dispatch kernel");
    });
}

// Stream s waits for what the side stream has queued so far.
hipError_t join_side(moe_ctx *ctx, hipStream_t s) {
    std::lock_guard<std::mutex> g(ctx->side_mu);
    hipError_t e = hipEventRecord(ctx->ev_join, ctx->side);
    return e == hipSuccess ? hipStreamWaitEvent(s, ctx->ev_join, 0) : e;
}
// x's encoding on the side stream: fork the side stream from s, encode x
// there (pieces for the MFMA and streaming kernels, int8 codes for the
// few-tokens kernels) and mark its end with ev_x, all before the routing is
// queued on s, so that the two run together.  wait_x then makes s wait for
// that mark before the first expert kernel.  A later call may record ev_x
// again before this call's wait_x; the side stream runs in order, so s then
// waits for a later point of it, which includes this call's encoding.
hipError_t encode_x_beside(moe_ctx *ctx, hipStream_t s, bool codes, const float *x, int t, int H, Workspace &w) {
    std::lock_guard<std::mutex> g(ctx->side_mu);
    hipError_t e = hipEventRecord(ctx->ev_fork, s);
    if (e == hipSuccess) e = hipStreamWaitEvent(ctx->side, ctx->ev_fork, 0);
    if (e == hipSuccess)
        e = codes ? launch_qenc(x, t, H, w.xq, ctx->side) : launch_split_rows(x, t, H, w.xhi, w.xlo, w.xex, ctx->side);
    return e == hipSuccess ? hipEventRecord(ctx->ev_x, ctx->side) : e;
}
hipError_t wait_x(moe_ctx *ctx, hipStream_t s) {
    std::lock_guard<std::mutex> g(ctx->side_mu);
    return hipStreamWaitEvent(s, ctx->ev_x, 0);
}

// The routed layer on workspace w (sized for at least t tokens of c.k
// experts).
int forward_on(moe_layer *L, const CallState &c, Workspace &w, const float *x, int t, float *out, float *residual,
               moe_route *routes, uint32_t *hits, const uint32_t *prev, uint64_t *stats, hipStream_t s) {
    const int k = c.k;
    // Path: the one-token kernels for one token, the few-tokens kernels
    // while experts hold few tokens each, MFMA beyond (it beats the register
    // GEMV at every size measured on MI355X), GEMV where the MFMA kernel does
    // not take the shapes, the exact kernels when neither fits (or when
    // asked).
    Path path = kExact;
    if (c.mode) {
        path = (Path)c.mode;
    } else if (L->fast_ok) {
        path = L->mfma_ok ? kMfma : kGemv;
        // The tiled copies' 32-token tiles beat the few-tokens kernels down
        // to half a token per expert on average (below it, each hit expert
        // holds about one token, which the integer-dot kernels stream faster).
        const bool tiled = L->tiled_mem && stream_tile((double)t * k / L->E, L->mfma_bm != 160) == 32;
        const bool batch = L->batch_ok && batch_pays(t, k, L->E, L->H, batch_tile_tokens(L->H, t, k, L->E));
        if (t == 1 && L->decode_ok)
            path = kDecode;
        else if (tiled && (!batch || 2 * t * k >= L->E))
            path = kStream;
        else if (batch)
            path = kBatch;
    }
    if (path == kBatch && (!L->batch_ok || t > w.batch_t)) path = L->mfma_ok ? kMfma : kGemv;
    if (path == kDecode) {
        const int dt_r = L->experts_host[0].m[0].dt;
        const int dt_s = L->has_shared ? L->experts_host[L->E].m[0].dt : dt_r;
        if (t != 1 || !L->decode_ok || !decode_fits(L->I, L->I_s, k, L->has_shared, dt_r, dt_s)) path = kGemv;
    }
    if (path == kStream && !L->mfma_ok) path = kGemv;
    if ((path == kMfma || path == kStream) && !mfma_fits(t, k, L->H, L->I, L->has_shared ? L->I_s : 0)) path = kGemv;
    const int bm = path == kMfma     ? mfma_call_tile(L->mfma_bm, t, k, L->E)
                   : path == kStream ? stream_tile((double)t * k / L->E, L->mfma_bm != 160)
                   : path == kBatch  ? batch_tile_tokens(L->H, t, k, L->E)
                                     : 0;
    const ExpertDev &e0 = L->experts_host[0];
    const ExpertDev *sh = L->has_shared ? &L->experts_host[L->E] : nullptr;
    // The shared expert on the context's side stream (few-tokens and MFMA
    // paths): x is encoded there while s routes, the shared expert then runs
    // there beside the routed experts, and it is joined back before the
    // combine.  Measured on MI355X against forking after the routing:
    // Qwen2-MoE T=32 0.197 -> 0.175 ms, T=512 0.424 -> 0.410, V2-Lite T=256
    // 0.348 -> 0.330.  Layers without a shared expert keep x's encoding on
    // s: the cross-stream wait costs more than the encoding (Mixtral T=32
    // 0.262 -> 0.273 ms with it beside).  Not while stages are being timed
    // on s, nor for the no-allocation entry, nor while s is being captured
    // into a graph (the capture then holds one stream's launches only).
    bool side = sh && c.side && !c.profile && L->ctx->side && (path == kBatch || path == kMfma || path == kStream);
    if (side && s) {
        hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
        if (hipStreamIsCapturing(s, &cs) != hipSuccess) {
            (void)hipGetLastError();  // the launches below report their own errors
            side = false;
        } else if (cs != hipStreamCaptureStatusNone) {
            side = false;
        }
    }
    hipError_t e = hipSuccess;
    if (side && (e = encode_x_beside(L->ctx, s, path == kBatch, x, t, L->H, w)) != hipSuccess)
        return hip_fail(e, "activation encoding (side stream)");
    int rc = route_and_dispatch(L, c, w, x, t, bm, path == kDecode, routes, hits, prev, stats, nullptr, s);
    if (rc) return rc;
    int ksplit = 1;
    if (path == kDecode) {
        DecodeArgs d{};
        d.tasks = w.dtasks;
        d.hits = w.hits;
        d.h = w.h;
        d.hs = w.hs;
        d.has_gate = L->has_shared_gate ? 1 : 0;
        d.out = out;
        d.residual = residual;
        d.H = L->H;
        d.I = L->I;
        d.I_s = L->I_s;
        d.E = L->E;
        d.k_bound = k;
        d.n_shared = L->has_shared ? 1 : 0;
        d.hq = w.dq;
        d.hq_units = std::max(L->I, L->has_shared ? L->I_s : 0) / 64;
        d.ys = w.ys;  // the shared expert's output when its down launch is separate
        const int dt_r = e0.m[0].dt, dt_s = sh ? sh->m[0].dt : dt_r;
        bool encoded = false;
        rc = stage(L, c.profile, 3, s, [&] {
            e = launch_decode_up(d, x, dt_r, dt_s, encoded, s);
            return e == hipSuccess ? MOE_OK : hip_fail(e, "one-token gate/up kernel");
        });
        if (rc) return rc;
        if (!encoded) {
            rc = stage(L, c.profile, 6, s, [&] {
                e = launch_decode_encode(d, s);
                return e == hipSuccess ? MOE_OK : hip_fail(e, "one-token encoding of h");
            });
            if (rc) return rc;
        }
        return stage(L, c.profile, 4, s, [&] {
            e = launch_decode_down(d, dt_r, dt_s, s);
            return e == hipSuccess ? MOE_OK : hip_fail(e, "one-token down kernel");
        });
    }
    if (path == kBatch) {
        BatchArgs b{};
        b.experts = L->experts_dev;
        b.tiles = w.tiles;
        b.ntiles = w.ntiles;
        b.counts = w.counts;
        b.offsets = w.offsets;
        b.perm_tok = w.perm_tok;
        b.xq = w.xq;
        b.h = w.h;
        b.hs = w.hs;
        b.hq = w.hq;
        b.hsq = w.hsq;
        b.y = w.y;
        b.ys = w.ys;
        b.T = t;
        b.H = L->H;
        b.I = L->I;
        b.I_s = L->I_s;
        b.E = L->E;
        b.max_tiles = t * k / bm + std::min(L->E, t * k) + 1;
        b.shared_tiles = L->has_shared ? (t + bm - 1) / bm : 0;
        b.ypart = (size_t)t * k * L->H;
        b.yspart = (size_t)t * L->H;
        b.ksplit = batch_ksplit(L->I, L->has_shared ? L->I_s : 0);
        b.nt = bm;
        if ((size_t)b.ksplit * t * k > w.y_rows || (size_t)b.ksplit * t > w.ys_rows)
            return fail(MOE_EUNSUP, "few-tokens path: %d K parts do not fit the workspace", b.ksplit);
        ksplit = b.ksplit;
        if (side) {
            if ((e = wait_x(L->ctx, s)) != hipSuccess) return hip_fail(e, "activation encoding (wait)");
        } else {
            rc = stage(L, c.profile, 6, s, [&] {
                e = launch_qenc(x, t, L->H, w.xq, s);
                return e == hipSuccess ? MOE_OK : hip_fail(e, "activation encoding");
            });
            if (rc) return rc;
        }
        if (side) {
            // The shared expert (its own buffers: hs, hsq, ys) beside the
            // routed experts, after x's encoding on the side stream; the
            // combine waits for both.
            e = launch_batch_up_shared(b, *sh, L->ctx->side);
            if (e == hipSuccess) e = launch_qenc(w.hs, t, L->I_s, w.hsq, L->ctx->side);
            if (e == hipSuccess) e = launch_batch_down_shared(b, *sh, L->ctx->side);
            if (e != hipSuccess) return hip_fail(e, "shared expert (few-tokens kernels)");
        }
        const ExpertDev *shs = side ? nullptr : sh;  // the shared expert on stream s
        rc = stage(L, c.profile, 3, s, [&] {
            e = launch_batch_up(b, e0, shs, s);
            return e == hipSuccess ? MOE_OK : hip_fail(e, "few-tokens gate/up kernel");
        });
        if (rc) return rc;
        rc = stage(L, c.profile, 6, s, [&] {
            e = launch_qenc(w.h, t * k, L->I, w.hq, s);
            if (e == hipSuccess && shs) e = launch_qenc(w.hs, t, L->I_s, w.hsq, s);
            return e == hipSuccess ? MOE_OK : hip_fail(e, "activation encoding");
        });
        if (rc) return rc;
        rc = stage(L, c.profile, 4, s, [&] {
            e = launch_batch_down(b, e0, shs, s);
            return e == hipSuccess ? MOE_OK : hip_fail(e, "few-tokens down kernel");
        });
        if (rc) return rc;
        if (side && (e = join_side(L->ctx, s)) != hipSuccess) return hip_fail(e, "shared expert join");
    } else if (path == kMfma || path == kStream) {
        const bool sp = path == kStream;
        MfmaArgs m{};
        m.experts = L->experts_dev;
        m.tiles = w.tiles;
        m.ntiles = w.ntiles;
        m.counts = w.counts;
        m.offsets = w.offsets;
        m.perm_tok = w.perm_tok;
        m.xhi = w.xhi;
        m.xlo = w.xlo;
        m.xex = w.xex;
        m.h = w.h;
        m.hs = w.hs;
        m.hhi = w.hhi;
        m.hlo = w.hlo;
        m.hex = w.hex;
        m.hshi = w.hshi;
        m.hslo = w.hslo;
        m.hsex = w.hsex;
        m.y = w.y;
        m.ys = w.ys;
        m.tail_part = w.tail_part;
        m.tail_cnt = w.tail_cnt;
        m.T = t;
        m.H = L->H;
        m.I = L->I;
        m.I_s = L->I_s;
        m.E = L->E;
        m.k = k;
        // Routed tiles: sum over experts of ceil(n_e / bm) <= t k / bm +
        // (experts with tokens); the shared expert's tiles follow them.
        m.max_tiles = t * k / bm + std::min(L->E, t * k) + 1;
        m.shared_tiles = L->has_shared ? (t + bm - 1) / bm : 0;
        m.ypart = (size_t)t * k * L->H;
        m.yspart = (size_t)t * L->H;
        m.ksplit = mfma_down_ksplit((t * k + bm - 1) / bm + std::min(L->E, t * k) / 2, L->H, L->I,
                                    L->has_shared ? L->I_s : 0);
        while (m.ksplit > 1 && ((size_t)m.ksplit * t * k > w.y_rows || (size_t)m.ksplit * t > w.ys_rows))
            m.ksplit /= 2;
        ksplit = m.ksplit;
        if (side) {
            if ((e = wait_x(L->ctx, s)) != hipSuccess) return hip_fail(e, "activation pieces (wait)");
        } else {
            rc = stage(L, c.profile, 6, s, [&] {
                e = launch_split_rows(x, t, L->H, w.xhi, w.xlo, w.xex, s);
                return e == hipSuccess ? MOE_OK : hip_fail(e, "activation pieces");
            });
            if (rc) return rc;
        }
        if (side) {
            // After x's pieces on the side stream.
            const int bs = sp ? stream_tile_exact(t, L->mfma_bm != 160) : bm;
            e = sp ? launch_stream_single(true, m, bs, *sh, L->ctx->side) : launch_mfma_single(true, m, bm, *sh, L->ctx->side);
            if (e == hipSuccess) e = launch_split_rows(w.hs, t, L->I_s, w.hshi, w.hslo, w.hsex, L->ctx->side);
            if (e == hipSuccess)
                e = sp ? launch_stream_single(false, m, bs, *sh, L->ctx->side) : launch_mfma_single(false, m, bm, *sh, L->ctx->side);
            if (e != hipSuccess) return hip_fail(e, "shared expert (MFMA kernels)");
        }
        const ExpertDev *shs = side ? nullptr : sh;
        rc = stage(L, c.profile, 3, s, [&] {
            e = sp ? launch_stream(true, m, bm, e0, shs, s) : launch_mfma(true, m, bm, e0, shs, s);
            return e == hipSuccess ? MOE_OK : hip_fail(e, "MFMA up kernel");
        });
        if (rc) return rc;
        rc = stage(L, c.profile, 6, s, [&] {
            e = launch_split_rows(w.h, t * k, L->I, w.hhi, w.hlo, w.hex, s);
            if (e == hipSuccess && shs) e = launch_split_rows(w.hs, t, L->I_s, w.hshi, w.hslo, w.hsex, s);
            return e == hipSuccess ? MOE_OK : hip_fail(e, "activation pieces");
        });
        if (rc) return rc;
        rc = stage(L, c.profile, 4, s, [&] {
            e = sp ? launch_stream(false, m, bm, e0, shs, s) : launch_mfma(false, m, bm, e0, shs, s);
            return e == hipSuccess ? MOE_OK : hip_fail(e, "MFMA down kernel");
        });
        if (rc) return rc;
        if (side && (e = join_side(L->ctx, s)) != hipSuccess) return hip_fail(e, "shared expert join");
    } else {
        GemvArgs a{};
        a.experts = L->experts_dev;
        a.hits = w.hits;
        a.counts = w.counts;
        a.offsets = w.offsets;
        a.perm_tok = w.perm_tok;
        a.x = x;
        a.h = w.h;
        a.hs = w.hs;
        a.y = w.y;
        a.ys = w.ys;
        a.T = t;
        a.H = L->H;
        a.I = L->I;
        a.I_s = L->I_s;
        a.E = L->E;
        a.task_bound = std::min(L->E, t * k);
        a.has_shared = L->has_shared;
        a.perm_w = w.perm_w;
        a.shgate = L->has_shared_gate ? w.shgate : nullptr;
        a.out = out;
        a.residual = residual;
        const bool fast = path == kGemv;
        rc = stage(L, c.profile, 3, s, [&] {
            e = fast ? launch_gemv_up(a, e0, sh, s) : launch_gemv_exact(true, a, s);
            return e == hipSuccess ? MOE_OK : hip_fail(e, "expert gate/up kernel");
        });
        if (rc) return rc;
        // Few tokens: the down projection performs the combine, the shared
        // expert and the residual add itself.
        const bool fused = fast && t <= kFusedMaxT;
        rc = stage(L, c.profile, 4, s, [&] {
            e = fast ? (fused ? launch_gemv_down_combine(a, e0, sh, s) : launch_gemv_down(a, e0, sh, s))
                     : launch_gemv_exact(false, a, s);
            return e == hipSuccess ? MOE_OK : hip_fail(e, "expert down kernel");
        });
        if (rc || fused) return rc;
    }
    CombineArgs cb{};
    cb.y = w.y;
    cb.ys = w.ys;
    cb.parts = ksplit;
    cb.ypart = (size_t)t * k * L->H;
    cb.yspart = (size_t)t * L->H;
    cb.pos = w.pos;
    cb.sel = w.sel;
    cb.wsel = w.wsel;
    cb.shgate = L->has_shared_gate ? w.shgate : nullptr;
    cb.out = out;
    cb.residual = residual;
    cb.T = t;
    cb.H = L->H;
    cb.k = k;
    cb.has_shared = L->has_shared;
    return stage(L, c.profile, 5, s, [&] {
        e = launch_combine(cb, s);
        return e == hipSuccess ? MOE_OK : hip_fail(e, "combine kernel");
    });
}

// ---- the allocation-free entry point -------------------------------------
// moe_layer_forward_noalloc runs on this array: device memory the code
// object itself carries, so no call allocates.  In host code `scratch` is
// only a stand-in for the symbol, never a device address: every host use
// goes through the per-device address hipGetSymbolAddress returns.  The
// counters at its start are zero at load (static storage) and every call
// leaves them at zero again; set-up clears them once more.  Every call on a
// device shares that device's array, so calls that overlap on one device
// race.
constexpr size_t kScratchBytes = (size_t)64 << 20;
constexpr int kMaxDevices = 64;
static __device__ __align__(256) uint8_t scratch[kScratchBytes];

std::mutex g_scratch_mu;
void *g_scratch_ptr[kMaxDevices] = {};

// The device address of `scratch` on `device` (which is current), looked up
// and cleared once per device.
int scratch_on(int device, void *&out) {
    if (device < 0 || device >= kMaxDevices) return fail(MOE_EUNSUP, "device %d: at most %d devices", device, kMaxDevices);
    std::lock_guard<std::mutex> g(g_scratch_mu);
    if (!g_scratch_ptr[device]) {
        void *p = nullptr;
        hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return hip_fail(e, "hipGetSymbolAddress(scratch)");
        if (!p || (uintptr_t)p % 256) return fail(MOE_EHIP, "scratch array at %p is not 256-byte aligned", p);
        if ((e = hipMemset(p, 0, kZeroBytes)) != hipSuccess) return hip_fail(e, "clearing the scratch counters");
        g_scratch_ptr[device] = p;
    }
    out = g_scratch_ptr[device];
    return MOE_OK;
}

// A caller's workspace laid out for t tokens of k experts, after checking
// that it is big enough.
int caller_ws(const moe_layer *L, int t, int k, void *ws, uint64_t ws_bytes, Workspace &w) {
    if (!ws) return fail(MOE_EINVAL, "workspace is NULL");
    if ((uintptr_t)ws % 256) return fail(MOE_EINVAL, "workspace is not 256-byte aligned");
    const size_t need = ws_layout(L, t, k, nullptr, nullptr);
    if (need > ws_bytes)
        return fail(MOE_EINVAL, "%d tokens of %d experts need a %zu-byte workspace; %llu given", t, k, need,
                    (unsigned long long)ws_bytes);
    ws_layout(L, t, k, &w, static_cast<char *>(ws));
    return MOE_OK;
}

}  // namespace

extern "C" {

const char *moe_last_error(void) { return g_err.c_str(); }

int moe_debug_expf(const float *x, float *y, uint64_t n, void *stream) {
    if ((!x || !y) && n) return fail(MOE_EINVAL, "moe_debug_expf: bad argument");
    hipError_t e = launch_expf(x, y, (size_t)n, (hipStream_t)stream);
    return e == hipSuccess ? MOE_OK : hip_fail(e, "expf kernel");
}

int moe_ctx_create(int device, moe_ctx **out) {
    if (!out) return fail(MOE_EINVAL, "moe_ctx_create: out is NULL");
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    if (e != hipSuccess) return hip_fail(e, "hipGetDeviceCount");
    if (device < 0 || device >= n) return fail(MOE_EINVAL, "device %d does not exist (%d visible)", device, n);
    auto *c = new moe_ctx();
    c->device = device;
    {
        DeviceGuard g(device);
        if (hipStreamCreateWithFlags(&c->side, hipStreamNonBlocking) != hipSuccess ||
            hipEventCreateWithFlags(&c->ev_fork, hipEventDisableTiming) != hipSuccess ||
            hipEventCreateWithFlags(&c->ev_join, hipEventDisableTiming) != hipSuccess ||
            hipEventCreateWithFlags(&c->ev_x, hipEventDisableTiming) != hipSuccess) {
            (void)hipGetLastError();
            c->side = nullptr;  // everything on the caller's stream
        }
    }
    *out = c;
    return MOE_OK;
}

void moe_ctx_destroy(moe_ctx *ctx) {
    if (!ctx) return;
    DeviceGuard g(ctx->device);
    hipDeviceSynchronize();
    for (auto &r : ctx->regions)
        if (r.ptr) hipFree(r.ptr);
    if (ctx->ev_fork) hipEventDestroy(ctx->ev_fork);
    if (ctx->ev_join) hipEventDestroy(ctx->ev_join);
    if (ctx->ev_x) hipEventDestroy(ctx->ev_x);
    if (ctx->side) hipStreamDestroy(ctx->side);
    delete ctx;
}

int moe_upload(moe_ctx *ctx, const void *host, uint64_t bytes, uint64_t *region_out) {
    if (!ctx || (!host && bytes) || !region_out) return fail(MOE_EINVAL, "moe_upload: bad argument");
    DeviceGuard g(ctx->device);
    void *p = nullptr;
    hipError_t e = hipMalloc(&p, std::max<uint64_t>(align_up(bytes, 256), 256));
    if (e != hipSuccess) return fail(MOE_ENOMEM, "moe_upload: %llu bytes: %s", (unsigned long long)bytes, hipGetErrorString(e));
    if (bytes) {
        e = hipMemcpy(p, host, bytes, hipMemcpyHostToDevice);
        if (e != hipSuccess) {
            hipFree(p);
            return hip_fail(e, "moe_upload: hipMemcpy");
        }
    }
    std::lock_guard<std::mutex> lk(ctx->mu);
    ctx->regions.push_back(Region{p, bytes});
    *region_out = ctx->regions.size() - 1;
    return MOE_OK;
}

int moe_upload_tensors(moe_ctx *ctx, const void *host, uint64_t host_len, const uint64_t *offsets,
                       const uint64_t *lengths, int64_t n, uint64_t *dev_offsets_out, uint64_t *region_out) {
    if (!ctx || !region_out || n < 0 || (n > 0 && (!host || !offsets || !lengths || !dev_offsets_out)))
        return fail(MOE_EINVAL, "moe_upload_tensors: bad argument");
    uint64_t total = 0;
    for (int64_t i = 0; i < n; i++) {
        if (offsets[i] > host_len || lengths[i] > host_len - offsets[i])
            return fail(MOE_EINVAL, "moe_upload_tensors: tensor %lld (%llu bytes at %llu) is outside the %llu-byte buffer",
                        (long long)i, (unsigned long long)lengths[i], (unsigned long long)offsets[i],
                        (unsigned long long)host_len);
        dev_offsets_out[i] = total;
        total = align_up(total + lengths[i], 256);
    }
    DeviceGuard g(ctx->device);
    void *p = nullptr;
    hipError_t e = hipMalloc(&p, std::max<uint64_t>(total, 256));
    if (e != hipSuccess)
        return fail(MOE_ENOMEM, "moe_upload_tensors: %llu bytes: %s", (unsigned long long)total, hipGetErrorString(e));
    for (int64_t i = 0; i < n; i++) {
        if (!lengths[i]) continue;
        e = hipMemcpy(static_cast<char *>(p) + dev_offsets_out[i], static_cast<const char *>(host) + offsets[i],
                      lengths[i], hipMemcpyHostToDevice);
        if (e != hipSuccess) {
            hipFree(p);
            return hip_fail(e, "moe_upload_tensors: hipMemcpy");
        }
    }
    std::lock_guard<std::mutex> lk(ctx->mu);
    ctx->regions.push_back(Region{p, total});
    *region_out = ctx->regions.size() - 1;
    return MOE_OK;
}

int moe_region_ptr(moe_ctx *ctx, uint64_t region, void **dev_out) {
    if (!ctx || !dev_out) return fail(MOE_EINVAL, "moe_region_ptr: bad argument");
    std::lock_guard<std::mutex> lk(ctx->mu);
    const Region *r = region_of(ctx, region);
    if (!r) return fail(MOE_EINVAL, "moe_region_ptr: unknown region %llu", (unsigned long long)region);
    *dev_out = r->ptr;
    return MOE_OK;
}

int moe_layer_create(moe_ctx *ctx, const moe_layer_desc *d, moe_layer **out) {
    if (!ctx || !d || !out) return fail(MOE_EINVAL, "moe_layer_create: bad argument");
    if (d->hidden <= 0 || d->n_experts <= 0 || d->top_k <= 0)
        return fail(MOE_EINVAL, "moe_layer_create: hidden %d, experts %d, top_k %d", d->hidden, d->n_experts, d->top_k);
    if (d->n_experts > kMaxExperts) return fail(MOE_EUNSUP, "%d experts; at most %d are supported", d->n_experts, kMaxExperts);
    if (std::min(d->top_k, d->n_experts) > kMaxTopK) return fail(MOE_EUNSUP, "top_k %d; at most %d is supported", d->top_k, kMaxTopK);
    if (d->n_group < 1 || d->topk_group < 0 || d->n_group > 64)
        return fail(MOE_EINVAL, "n_group %d, topk_group %d", d->n_group, d->topk_group);
    if (d->gate != MOE_GATE_SOFTMAX && d->gate != MOE_GATE_SIGMOID) return fail(MOE_EINVAL, "gate kind %d", d->gate);
    if (!d->experts) return fail(MOE_EINVAL, "moe_layer_create: experts is NULL");
    DeviceGuard g(ctx->device);
    std::lock_guard<std::mutex> lk(ctx->mu);
    auto L = std::make_unique<moe_layer>();
    L->ctx = ctx;
    L->H = d->hidden;
    L->E = d->n_experts;
    L->top_k_spec = d->top_k;
    L->gate = d->gate;
    L->norm_topk = d->norm_topk;
    L->n_group = d->n_group;
    L->topk_group = d->topk_group;
    L->routed_scale = d->routed_scale;
    const int H = L->H, E = L->E;

    MatDev router;
    int rc = resolve(ctx, d->router, E, H, "router", router);
    if (rc) return rc;
    if (router.dt != MOE_DT_F32) return fail(MOE_EUNSUP, "router: only F32 routers are supported");
    MatDev sg{};
    L->has_shared_gate = present(d->shared_gate);
    if (L->has_shared_gate) {
        if ((rc = resolve(ctx, d->shared_gate, 1, H, "shared_gate", sg))) return rc;
        if (sg.dt != MOE_DT_F32) return fail(MOE_EUNSUP, "shared_gate: only F32 is supported");
    }
    if (present(d->e_bias)) {
        MatDev b;
        if ((rc = resolve(ctx, d->e_bias, 1, E, "e_bias", b))) return rc;
        if (b.dt != MOE_DT_F32) return fail(MOE_EUNSUP, "e_bias: only F32 is supported");
        if ((uintptr_t)b.ptr % 4) return fail(MOE_EINVAL, "e_bias: not 4-byte aligned");
        L->e_bias = reinterpret_cast<const float *>(b.ptr);
    }

    // Experts.
    L->experts_host.resize(E + 1);
    int I = -1;
    for (int e = 0; e < E; e++) {
        const moe_tensor *t = d->experts + 3 * e;
        const int inter = t[0].rows;
        if (inter <= 0) return fail(MOE_EINVAL, "expert %d: %d rows", e, inter);
        if (I < 0) I = inter;
        if (inter != I) return fail(MOE_EUNSUP, "expert %d: intermediate %d differs from expert 0's %d", e, inter, I);
        char what[64];
        ExpertDev &x = L->experts_host[e];
        snprintf(what, sizeof what, "expert %d gate", e);
        if ((rc = resolve(ctx, t[0], inter, H, what, x.m[0]))) return rc;
        snprintf(what, sizeof what, "expert %d up", e);
        if ((rc = resolve(ctx, t[1], inter, H, what, x.m[1]))) return rc;
        snprintf(what, sizeof what, "expert %d down", e);
        if ((rc = resolve(ctx, t[2], H, inter, what, x.m[2]))) return rc;
        x.inter = inter;
    }
    L->I = I;
    L->has_shared = present(d->shared[0]);
    if (L->has_shared) {
        const int inter = d->shared[0].rows;
        ExpertDev &x = L->experts_host[E];
        if ((rc = resolve(ctx, d->shared[0], inter, H, "shared gate_proj", x.m[0]))) return rc;
        if ((rc = resolve(ctx, d->shared[1], inter, H, "shared up_proj", x.m[1]))) return rc;
        if ((rc = resolve(ctx, d->shared[2], H, inter, "shared down_proj", x.m[2]))) return rc;
        x.inter = inter;
        L->I_s = inter;
    }

    // Which kernels the shapes allow.
    const ExpertDev &e0 = L->experts_host[0];
    bool fast = true;
    for (int e = 0; e < E; e++)
        for (int m = 0; m < 3; m++) {
            const MatDev &a = L->experts_host[e].m[m], &b = e0.m[m];
            fast &= fast_mat(a) && a.dt == b.dt && a.dt != MOE_DT_F32;
        }
    fast &= e0.m[0].dt == e0.m[1].dt;
    if (L->has_shared) {
        const ExpertDev &s = L->experts_host[E];
        for (int m = 0; m < 3; m++) fast &= fast_mat(s.m[m]) && s.m[m].dt != MOE_DT_F32;
        fast &= s.m[0].dt == s.m[1].dt;
    }
    L->fast_ok = fast;
    bool fmt = true;
    for (int e = 0; e < E + (L->has_shared ? 1 : 0); e++)
        for (int m = 0; m < 3; m++) {
            const MatDev &mm = L->experts_host[e].m[m];
            fmt &= mfma_format_ok(mm.dt) && (size_t)mm.rows * mm.stride < ((size_t)1 << 32);
        }
    L->mfma_ok = fast && fmt && H % 64 == 0 && I % 64 == 0 && (!L->has_shared || L->I_s % 64 == 0);
    L->decode_ok = fast && decode_supported(H, I, L->has_shared ? L->I_s : 0, e0.m[0].dt,
                                            L->has_shared ? L->experts_host[E].m[0].dt : e0.m[0].dt);
    if (L->has_shared) {
        const ExpertDev &s = L->experts_host[E];
        L->decode_ok &= s.m[0].dt == s.m[2].dt;
    }
    L->decode_ok &= e0.m[0].dt == e0.m[2].dt;
    L->batch_ok = fast && batch_supported(H, I, L->has_shared ? L->I_s : 0, e0.m[0].dt,
                                          L->has_shared ? L->experts_host[E].m[0].dt : e0.m[0].dt);
    for (int e = 0; e < E + (L->has_shared ? 1 : 0); e++) L->batch_ok &= batch_supported(H, I, 0, L->experts_host[e].m[2].dt, 0);

    // Device-side tables.
    hipError_t he;
    const int n_rows = E + (L->has_shared_gate ? 1 : 0);
    if ((he = hipMalloc(&L->router, (size_t)n_rows * H * 4)) != hipSuccess) return hip_fail(he, "router copy");
    if ((he = hipMemcpy(L->router, router.ptr, (size_t)E * H * 4, hipMemcpyDeviceToDevice)) != hipSuccess)
        return hip_fail(he, "router copy");
    if (L->has_shared_gate &&
        (he = hipMemcpy(L->router + (size_t)E * H, sg.ptr, (size_t)H * 4, hipMemcpyDeviceToDevice)) != hipSuccess)
        return hip_fail(he, "shared gate copy");
    if ((he = hipMalloc(&L->experts_dev, sizeof(ExpertDev) * (E + 1))) != hipSuccess) return hip_fail(he, "expert table");
    if ((he = hipMemcpy(L->experts_dev, L->experts_host.data(), sizeof(ExpertDev) * (E + 1), hipMemcpyHostToDevice)) !=
        hipSuccess)
        return hip_fail(he, "expert table");
    std::vector<unsigned long long> eb(E);
    for (int e = 0; e < E; e++) {
        const ExpertDev &x = L->experts_host[e];
        for (int m = 0; m < 3; m++) eb[e] += (unsigned long long)moe_row_bytes(x.m[m].dt, x.m[m].cols) * x.m[m].rows;
    }
    if ((he = hipMalloc(&L->expert_bytes, 8 * E)) != hipSuccess) return hip_fail(he, "expert bytes");
    if ((he = hipMemcpy(L->expert_bytes, eb.data(), 8 * E, hipMemcpyHostToDevice)) != hipSuccess)
        return hip_fail(he, "expert bytes");
    if (L->mfma_ok) {
        // Per matrix, the power of two that puts the largest |d q| in
        // [2^14, 2^15) for the MFMA path's f16 pieces (|q| <= 8, 16, 128).
        const int n = E + (L->has_shared ? 1 : 0);
        unsigned *mx = nullptr;
        std::vector<unsigned> host(3 * (size_t)n, 0u);
        if ((he = hipMalloc(&mx, 4 * host.size())) != hipSuccess) return hip_fail(he, "scale maxima");
        he = hipMemset(mx, 0, 4 * host.size());
        if (he == hipSuccess) he = launch_scale_max(L->experts_dev, n, mx, nullptr);
        if (he == hipSuccess) he = hipMemcpy(host.data(), mx, 4 * host.size(), hipMemcpyDeviceToHost);
        hipFree(mx);
        if (he != hipSuccess) return hip_fail(he, "scale maxima");
        for (int e = 0; e < n; e++)
            for (int m = 0; m < 3; m++) {
                MatDev &md = L->experts_host[e].m[m];
                const unsigned bits = host[3 * (size_t)e + m];
                const float qmax = md.dt == MOE_DT_Q4_0 ? 8.0f : md.dt == MOE_DT_Q5_0 ? 16.0f : 128.0f;
                md.wexp = 0;
                if (bits) {
                    int fe = 0;
                    (void)std::frexp(f16_bits_to_float(bits) * qmax, &fe);  // < 2^fe
                    md.wexp = 15 - fe;
                }
            }
        if ((he = hipMemcpy(L->experts_dev, L->experts_host.data(), sizeof(ExpertDev) * (E + 1),
                            hipMemcpyHostToDevice)) != hipSuccess)
            return hip_fail(he, "expert table");
        std::vector<int> dts;
        for (int e = 0; e < n; e++)
            for (int m = 0; m < 3; m++) dts.push_back(L->experts_host[e].m[m].dt);
        L->mfma_bm = mfma_tile_m(dts.data(), (int)dts.size());
    }
    *out = L.release();
    return MOE_OK;
}

void moe_layer_destroy(moe_layer *L) {
    if (!L) return;
    DeviceGuard g(L->ctx->device);
    hipDeviceSynchronize();
    for (StreamWs &e : L->ws) hipFree(e.w.base);
    for (Retired &r : L->retired) {
        hipFree(r.base);
        if (r.done) hipEventDestroy(r.done);
    }
    hipFree(L->tiled_mem);
    hipFree(L->router);
    hipFree(L->experts_dev);
    hipFree(L->expert_bytes);
    for (auto &r : L->pending) L->event_pool.push_back(r.a), L->event_pool.push_back(r.b);
    for (hipEvent_t ev : L->event_pool) hipEventDestroy(ev);
    delete L;
}

int moe_layer_set_routing(moe_layer *L, const moe_routing *r) {
    if (!L) return fail(MOE_EINVAL, "moe_layer_set_routing: layer is NULL");
    uint32_t dis[kMaxExperts / 32] = {};
    int32_t forced[kMaxForced] = {};
    int n_forced = 0;
    float temp = 0.0f;
    int top_k = 0;
    bool any = false;
    if (r) {
        if (r->n_disabled < 0 || r->n_forced < 0 || (r->n_disabled && !r->disabled) || (r->n_forced && !r->forced))
            return fail(MOE_EINVAL, "moe_layer_set_routing: bad lists");
        if (r->n_forced > kMaxForced) return fail(MOE_EUNSUP, "at most %d forced experts", kMaxForced);
        for (int i = 0; i < r->n_disabled; i++) {
            const int e = r->disabled[i];
            if (e >= 0 && e < L->E) dis[e >> 5] |= 1u << (e & 31), any = true;
        }
        for (int i = 0; i < r->n_forced; i++) forced[n_forced++] = r->forced[i];
        temp = r->temp;
        top_k = r->top_k;
        if (top_k < 0) return fail(MOE_EINVAL, "top_k %d", top_k);
        if (std::min(top_k, L->E) > kMaxTopK) return fail(MOE_EUNSUP, "top_k %d; at most %d is supported", top_k, kMaxTopK);
    }
    // Takes effect for calls made after this one; calls already queued keep
    // the routing they were launched with (it travels in their arguments).
    std::lock_guard<std::mutex> g(L->mu);
    std::memcpy(L->disabled, dis, sizeof dis);
    std::memcpy(L->forced, forced, sizeof forced);
    L->any_disabled = any;
    L->n_forced = n_forced;
    L->temp = temp;
    L->top_k_override = top_k;
    return MOE_OK;
}

int moe_layer_set_tiled(moe_layer *L, int enable) {
    if (!L) return fail(MOE_EINVAL, "moe_layer_set_tiled: bad argument");
    if (enable && !L->mfma_ok) return fail(MOE_EUNSUP, "this layer's shapes do not fit the MFMA kernels");
    DeviceGuard g(L->ctx->device);
    std::lock_guard<std::mutex> lk(L->mu);
    if ((L->tiled_mem != nullptr) == (enable != 0)) return MOE_OK;
    hipError_t he = hipDeviceSynchronize();  // queued calls may read the expert table
    if (he != hipSuccess) return hip_fail(he, "moe_layer_set_tiled");
    const int n = L->E + (L->has_shared ? 1 : 0);
    if (!enable) {
        for (int e = 0; e < n; e++)
            for (MatDev &m : L->experts_host[e].m) m.tiled = nullptr;
        he = hipMemcpy(L->experts_dev, L->experts_host.data(), sizeof(ExpertDev) * (L->E + 1), hipMemcpyHostToDevice);
        hipFree(L->tiled_mem);
        L->tiled_mem = nullptr;
        return he == hipSuccess ? MOE_OK : hip_fail(he, "expert table");
    }
    size_t total = 0;
    for (int e = 0; e < n; e++)
        for (const MatDev &m : L->experts_host[e].m) {
            const size_t b = tiled_bytes(m);
            if (!b) return fail(MOE_EUNSUP, "expert %d: a matrix's format or shape has no tiled layout", e);
            total += (b + 255) / 256 * 256;
        }
    uint8_t *mem = nullptr;
    if ((he = hipMalloc(&mem, total)) != hipSuccess)
        return fail(MOE_ENOMEM, "tiled expert copies (%zu bytes): %s", total, hipGetErrorString(he));
    size_t off = 0;
    std::vector<ExpertDev> table = L->experts_host;
    for (int e = 0; e < n && he == hipSuccess; e++)
        for (MatDev &m : table[e].m) {
            if ((he = tile_matrix(m, mem + off, nullptr)) != hipSuccess) break;
            m.tiled = mem + off;
            off += (tiled_bytes(m) + 255) / 256 * 256;
        }
    if (he == hipSuccess) he = hipDeviceSynchronize();
    if (he == hipSuccess)
        he = hipMemcpy(L->experts_dev, table.data(), sizeof(ExpertDev) * (L->E + 1), hipMemcpyHostToDevice);
    if (he != hipSuccess) {
        hipFree(mem);
        (void)hipMemcpy(L->experts_dev, L->experts_host.data(), sizeof(ExpertDev) * (L->E + 1),
                        hipMemcpyHostToDevice);
        return hip_fail(he, "tiled expert copies");
    }
    L->experts_host = table;
    L->tiled_mem = mem;
    return MOE_OK;
}

int moe_layer_set_mode(moe_layer *L, int mode) {
    if (!L || mode < 0 || mode > kStream) return fail(MOE_EINVAL, "moe_layer_set_mode: mode %d", mode);
    if (mode == kBatch && !L->batch_ok) return fail(MOE_EUNSUP, "this layer's shapes do not fit the few-tokens kernels");
    if (mode == kDecode && !L->decode_ok) return fail(MOE_EUNSUP, "this layer's shapes do not fit the one-token kernels");
    if (mode == kGemv && !L->fast_ok) return fail(MOE_EUNSUP, "this layer's shapes do not fit the GEMV kernels");
    if ((mode == kMfma || mode == kStream) && !L->mfma_ok)
        return fail(MOE_EUNSUP, "this layer's shapes do not fit the MFMA kernels");
    std::lock_guard<std::mutex> g(L->mu);
    L->mode = mode;
    return MOE_OK;
}

int moe_layer_reserve_stream(moe_layer *L, int32_t max_t, void *stream) {
    if (!L || max_t <= 0) return fail(MOE_EINVAL, "moe_layer_reserve: bad argument");
    DeviceGuard g(L->ctx->device);
    int k;
    {
        std::lock_guard<std::mutex> lk(L->mu);
        k = std::max(effective_k_locked(L), std::min(L->top_k_spec, L->E));
        L->reserved_t = std::max(L->reserved_t, (int)max_t);
        L->reserved_k = std::max(L->reserved_k, k);
    }
    Workspace w;
    return stream_ws(L, (hipStream_t)stream, max_t, k, w);
}

int moe_layer_reserve(moe_layer *L, int32_t max_t) { return moe_layer_reserve_stream(L, max_t, nullptr); }

int moe_layer_release_stream(moe_layer *L, void *stream) {
    if (!L) return fail(MOE_EINVAL, "moe_layer_release_stream: bad argument");
    DeviceGuard g(L->ctx->device);
    std::lock_guard<std::mutex> lk(L->mu);
    for (size_t i = 0; i < L->ws.size(); i++) {
        if (L->ws[i].stream != (hipStream_t)stream) continue;
        retire_ws(L, L->ws[i].w.base, L->ws[i].stream);
        L->ws.erase(L->ws.begin() + i);
        break;
    }
    reap_ws(L);
    return MOE_OK;
}

int moe_layer_k(const moe_layer *L) {
    if (!L) return 0;
    std::lock_guard<std::mutex> g(const_cast<moe_layer *>(L)->mu);
    return effective_k_locked(L);
}

int moe_layer_workspace_size(const moe_layer *L, int32_t max_t, uint64_t *bytes) {
    if (!L || max_t <= 0 || !bytes) return fail(MOE_EINVAL, "moe_layer_workspace_size: bad argument");
    *bytes = ws_layout(L, max_t, moe_layer_k(L), nullptr, nullptr);
    return MOE_OK;
}

int moe_layer_route(moe_layer *L, const float *x, int32_t t, moe_route *routes, float *logits, void *stream) {
    if (!L || !x || t <= 0) return fail(MOE_EINVAL, "moe_layer_route: bad argument");
    DeviceGuard g(L->ctx->device);
    hipStream_t s = (hipStream_t)stream;
    const CallState c = snapshot(L);
    Workspace w;
    int rc = stream_ws(L, s, t, c.k, w);
    if (rc) return rc;
    return route_and_dispatch(L, c, w, x, t, 0, false, routes, nullptr, nullptr, nullptr, logits, s);
}

int moe_debug_mfma_kernel(int32_t choice) {
    if (choice < 0 || choice > 1) return fail(MOE_EINVAL, "moe_debug_mfma_kernel: choice %d (0 or 1)", choice);
    return set_mfma_kernel(choice);
}

int moe_debug_decode_kernel(int32_t choice) {
    if (choice < 0 || choice > 2) return fail(MOE_EINVAL, "moe_debug_decode_kernel: choice %d (0, 1 or 2)", choice);
    return set_decode_kernel(choice);
}

int moe_layer_forward(moe_layer *L, const float *x, int32_t t, float *out, float *residual, moe_route *routes,
                      uint32_t *hits, const uint32_t *prev, uint64_t *stats, void *stream) {
    if (!L || !x || !out || t <= 0) return fail(MOE_EINVAL, "moe_layer_forward: bad argument (t = %d)", t);
    DeviceGuard g(L->ctx->device);
    hipStream_t s = (hipStream_t)stream;
    const CallState c = snapshot(L);
    Workspace w;
    int rc = stream_ws(L, s, t, c.k, w);
    if (rc) return rc;
    return forward_on(L, c, w, x, t, out, residual, routes, hits, prev, stats, s);
}

int moe_layer_forward_ws(moe_layer *L, const float *x, int32_t t, float *out, float *residual, moe_route *routes,
                         uint32_t *hits, const uint32_t *prev, uint64_t *stats, void *workspace,
                         uint64_t workspace_bytes, void *stream) {
    if (!L || !x || !out || t <= 0) return fail(MOE_EINVAL, "moe_layer_forward_ws: bad argument (t = %d)", t);
    DeviceGuard g(L->ctx->device);
    const CallState c = snapshot(L);
    Workspace w;
    int rc = caller_ws(L, t, c.k, workspace, workspace_bytes, w);
    if (rc) return rc;
    return forward_on(L, c, w, x, t, out, residual, routes, hits, prev, stats, (hipStream_t)stream);
}

int moe_layer_forward_noalloc(moe_layer *L, const float *x, int32_t t, float *out, float *residual,
                              moe_route *routes, uint32_t *hits, const uint32_t *prev, uint64_t *stats, void *stream) {
    if (!L || !x || !out || t <= 0) return fail(MOE_EINVAL, "moe_layer_forward_noalloc: bad argument (t = %d)", t);
    DeviceGuard g(L->ctx->device);
    CallState c = snapshot(L);
    c.profile = false;  // stage timing creates events; this entry point allocates nothing
    c.side = false;     // one stream: what a caller capturing or pinning its stream expects
    const size_t need = ws_layout(L, t, c.k, nullptr, nullptr);
    if (need > kScratchBytes)
        return fail(MOE_EINVAL,
                    "moe_layer_forward_noalloc: %d tokens of %d experts need %zu bytes of scratch; the static "
                    "array holds %zu (use moe_layer_forward_ws with a larger workspace)",
                    t, c.k, need, kScratchBytes);
    void *base = nullptr;
    int rc = scratch_on(L->ctx->device, base);
    if (rc) return rc;
    Workspace w;
    ws_layout(L, t, c.k, &w, static_cast<char *>(base));
    return forward_on(L, c, w, x, t, out, residual, routes, hits, prev, stats, (hipStream_t)stream);
}

}  // extern "C"

// ---- plain projections ------------------------------------------------------
// quant::matmul (src/quant.rs:482-506) for the weights around the routed
// layers: attention projections, the dense path's projections and lm_head.
// The matrix is held like a shared expert's down projection (table entry
// 0 = the matrix), so the expert kernels run it unchanged: the f32 GEMV for
// a few tokens, the MFMA kernel (f16 pieces, f32 accumulation) beyond, the
// exact kernel (the reference's dot, bit for bit) for formats and widths
// those do not take.
struct moe_linear {
    moe_ctx *ctx = nullptr;
    ExpertDev host{};
    ExpertDev *dev = nullptr;  // owned: freed with the object, also on a failed create
    bool fast = false, mfma = false;
    int bm = 160;
    ~moe_linear() {
        if (dev) hipFree(dev);
    }
};

namespace {

// Tokens up to which the GEMV beats the MFMA path for one matrix.
constexpr int kLinearGemvMaxT = 8;
constexpr size_t kLinearPartsMax = (size_t)32 << 20;  // bytes of K-split partial outputs

// K parts of one MFMA projection over t tokens.  A block walks its K range
// one ring step at a time (~1.5 µs per 64 values at one token tile), so a
// matrix of few 256-row tiles leaves the CUs idle and each block slow:
// measured on MI355X, V2-Lite's 2048 -> 3072 projection at T=32 took 50 µs
// in 12 blocks.  Split K (each part two steps or more) until the grid has
// 256 blocks; the parts are summed in order afterwards.
int linear_ksplit(const moe_linear *l, int t) {
    const MatDev &m = l->host.m[2];
    const long long blocks = (long long)((t + l->bm - 1) / l->bm) * ((m.rows + 255) / 256);
    int ks = 1;
    while (ks < 16 && blocks * ks < 256 && m.cols % (2 * ks * 64) == 0 && m.cols / (2 * ks) >= 128 &&
           (size_t)2 * ks * t * m.rows * 4 <= kLinearPartsMax)
        ks *= 2;
    return ks;
}

// Parts buffer for any t <= max_t: ks * t * rows floats, largest at the top
// of a run of t with the same number of token tiles.
size_t linear_parts_bytes(const moe_linear *l, int max_t) {
    size_t best = 0;
    for (int top = l->bm;; top += l->bm) {
        const int t = std::min(top, max_t);
        const int ks = linear_ksplit(l, t);
        if (ks > 1) best = std::max(best, (size_t)ks * t * l->host.m[2].rows * 4);
        if (top >= max_t) break;
    }
    return best;
}

size_t linear_ws_layout(const moe_linear *l, int max_t, char *base, uint16_t **hi, uint16_t **lo, int32_t **ex,
                        float **parts) {
    const size_t T = (size_t)max_t, K = (size_t)l->host.m[2].cols;
    const bool pieces = l->mfma && max_t > kLinearGemvMaxT;
    const size_t a = pieces ? align_up(T * K * 2, 256) : 0, b = pieces ? align_up(T * 4, 256) : 0;
    const size_t c = pieces ? align_up(linear_parts_bytes(l, max_t), 256) : 0;
    if (base && pieces) {
        *hi = reinterpret_cast<uint16_t *>(base);
        *lo = reinterpret_cast<uint16_t *>(base + a);
        *ex = reinterpret_cast<int32_t *>(base + 2 * a);
        *parts = c ? reinterpret_cast<float *>(base + 2 * a + b) : nullptr;
    }
    return std::max<size_t>(2 * a + b + c, 256);
}

}  // namespace

extern "C" {

int moe_linear_create(moe_ctx *ctx, const moe_tensor *w, moe_linear **out) {
    if (!ctx || !w || !out) return fail(MOE_EINVAL, "moe_linear_create: bad argument");
    if (w->rows <= 0 || w->cols <= 0) return fail(MOE_EINVAL, "moe_linear_create: shape [%d, %d]", w->rows, w->cols);
    DeviceGuard g(ctx->device);
    auto l = std::make_unique<moe_linear>();
    l->ctx = ctx;
    MatDev m;
    int rc;
    {
        std::lock_guard<std::mutex> lk(ctx->mu);
        rc = resolve(ctx, *w, w->rows, w->cols, "linear weight", m);
    }
    if (rc) return rc;
    l->host.m[0] = l->host.m[1] = l->host.m[2] = m;
    l->host.inter = m.cols;
    l->fast = fast_mat(m) && m.dt != MOE_DT_F32;
    l->mfma = l->fast && mfma_format_ok(m.dt) && m.cols % 64 == 0 && (size_t)m.rows * m.stride < ((size_t)1 << 32);
    hipError_t he;
    if ((he = hipMalloc(&l->dev, sizeof(ExpertDev))) != hipSuccess) return hip_fail(he, "linear table");
    if (l->mfma) {
        unsigned *mx = nullptr, host[3] = {0, 0, 0};
        if ((he = hipMemcpy(l->dev, &l->host, sizeof(ExpertDev), hipMemcpyHostToDevice)) != hipSuccess ||
            (he = hipMalloc(&mx, 12)) != hipSuccess)
            return hip_fail(he, "linear scale maxima");
        he = hipMemset(mx, 0, 12);
        if (he == hipSuccess) he = launch_scale_max(l->dev, 1, mx, nullptr);
        if (he == hipSuccess) he = hipMemcpy(host, mx, 12, hipMemcpyDeviceToHost);
        hipFree(mx);
        if (he != hipSuccess) return hip_fail(he, "linear scale maxima");
        const float qmax = m.dt == MOE_DT_Q4_0 ? 8.0f : m.dt == MOE_DT_Q5_0 ? 16.0f : 128.0f;
        int wexp = 0;
        if (host[2]) {
            int fe = 0;
            (void)std::frexp(f16_bits_to_float(host[2]) * qmax, &fe);
            wexp = 15 - fe;
        }
        for (int i = 0; i < 3; i++) l->host.m[i].wexp = wexp;
        const int dt = m.dt;
        l->bm = mfma_tile_m(&dt, 1);
    }
    if ((he = hipMemcpy(l->dev, &l->host, sizeof(ExpertDev), hipMemcpyHostToDevice)) != hipSuccess)
        return hip_fail(he, "linear table");
    *out = l.release();
    return MOE_OK;
}

void moe_linear_destroy(moe_linear *l) {
    if (!l) return;
    DeviceGuard g(l->ctx->device);
    hipDeviceSynchronize();
    delete l;
}

int moe_linear_workspace_size(const moe_linear *l, int32_t max_t, uint64_t *bytes) {
    if (!l || max_t <= 0 || !bytes) return fail(MOE_EINVAL, "moe_linear_workspace_size: bad argument");
    *bytes = linear_ws_layout(l, max_t, nullptr, nullptr, nullptr, nullptr, nullptr);
    return MOE_OK;
}

int moe_linear_forward(moe_linear *l, const float *x, int32_t t, float *y, float *residual, void *workspace,
                       uint64_t workspace_bytes, void *stream) {
    if (!l || !x || !y || t <= 0) return fail(MOE_EINVAL, "moe_linear_forward: bad argument (t = %d)", t);
    DeviceGuard g(l->ctx->device);
    hipStream_t s = (hipStream_t)stream;
    const MatDev &m = l->host.m[2];
    hipError_t e = hipSuccess;
    if (l->mfma && t > kLinearGemvMaxT) {
        const size_t need = linear_ws_layout(l, t, nullptr, nullptr, nullptr, nullptr, nullptr);
        if (!workspace || workspace_bytes < need || (uintptr_t)workspace % 256)
            return fail(MOE_EINVAL, "moe_linear_forward: %d tokens need a 256-byte-aligned workspace of %zu bytes", t,
                        need);
        uint16_t *hi = nullptr, *lo = nullptr;
        int32_t *ex = nullptr;
        float *parts = nullptr;
        linear_ws_layout(l, t, static_cast<char *>(workspace), &hi, &lo, &ex, &parts);
        const int ks = linear_ksplit(l, t);
        MfmaArgs a{};
        a.experts = l->dev;
        a.E = 0;
        a.T = t;
        a.H = m.rows;
        a.I = a.I_s = m.cols;
        a.hshi = hi;
        a.hslo = lo;
        a.hsex = ex;
        a.ys = ks > 1 ? parts : y;
        a.yspart = (size_t)t * m.rows;
        a.ksplit = ks;
        a.shared_tiles = (t + l->bm - 1) / l->bm;
        e = launch_split_rows(x, t, m.cols, hi, lo, ex, s);
        if (e == hipSuccess) e = launch_mfma_single(false, a, l->bm, l->host, s);
        if (e == hipSuccess && ks > 1) {
            // y = the parts summed in order; residual += y in the same pass.
            e = launch_sum_parts(parts, ks, (size_t)t * m.rows, y, residual, s);
            if (e != hipSuccess) return hip_fail(e, "linear K parts");
            return MOE_OK;
        }
    } else {
        GemvArgs a{};
        a.experts = l->dev;
        a.E = 0;
        a.T = t;
        a.H = m.rows;
        a.I = a.I_s = m.cols;
        a.hs = const_cast<float *>(x);
        a.ys = y;
        a.task_bound = 0;
        a.has_shared = 1;
        e = l->fast ? launch_gemv_down_single(a, l->host, s) : launch_gemv_exact(false, a, s);
    }
    if (e != hipSuccess) return hip_fail(e, "linear kernels");
    if (residual) {
        // residual += y, as the attention block's x += o(ctx) (src/model.rs:676-679).
        e = launch_add(residual, y, (size_t)t * m.rows, s);
        if (e != hipSuccess) return hip_fail(e, "residual add");
    }
    return MOE_OK;
}

int moe_layer_profile(moe_layer *L, int enable) {
    if (!L) return fail(MOE_EINVAL, "moe_layer_profile: layer is NULL");
    std::lock_guard<std::mutex> g(L->mu);
    L->profile = enable != 0;
    return MOE_OK;
}

int moe_layer_stage_times(moe_layer *L, double *ms, uint64_t *n) {
    if (!L || !ms || !n) return fail(MOE_EINVAL, "moe_layer_stage_times: bad argument");
    DeviceGuard g(L->ctx->device);
    std::lock_guard<std::mutex> lk(L->mu);
    if (!L->pending.empty()) {
        hipError_t e = hipEventSynchronize(L->pending.back().b);
        if (e != hipSuccess) return hip_fail(e, "hipEventSynchronize");
    }
    for (auto &r : L->pending) {
        float t = 0.0f;
        if (hipEventSynchronize(r.b) == hipSuccess && hipEventElapsedTime(&t, r.a, r.b) == hipSuccess) {
            L->stage_ms[r.stage] += t;
            L->stage_n[r.stage] += 1;
        }
        L->event_pool.push_back(r.a);
        L->event_pool.push_back(r.b);
    }
    L->pending.clear();
    for (int i = 0; i < MOE_STAGES; i++) {
        ms[i] += L->stage_ms[i];
        n[i] += L->stage_n[i];
        L->stage_ms[i] = 0.0;
        L->stage_n[i] = 0;
    }
    return MOE_OK;
}

}  // extern "C"
