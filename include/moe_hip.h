/*
 * moe_hip.h — C ABI of libmoe_hip, the MI355X (gfx950) routed-MoE layer.
 *
 * The reference (JGalego/Moe, a Rust crate) has no FFI: its boundary is the
 * internal call
 *     Model::feed_forward(&self, layer, li, x: &[f32], t, st: &mut State,
 *                         out: &mut [f32])            src/model.rs:836-841
 * whose Ffn::Moe arm (src/model.rs:841-971) routes, dispatches, runs the
 * SwiGLU experts over Q4_0/Q5_0/Q8_0 row ranges and combines.  Every entry
 * point below names the reference interface it replaces.  Plain C types only:
 * pointers, sizes and POD structs; no C++ or torch types cross this line.
 *
 * Conventions
 *   - Every function returns 0 on success or a negative MOE_E* code; the
 *     message of the most recent failure on the calling thread is returned by
 *     moe_last_error().
 *   - Device pointers are HIP device addresses on the context's device.
 *     `stream` is a hipStream_t passed as void* (NULL = the null stream).
 *   - A forward call is asynchronous on `stream` and never waits for the
 *     device.  Calls are reentrant per stream, as the reference's
 *     Model::feed_forward(&self, ..., st: &mut State, ...) is per sequence
 *     (src/model.rs:836): moe_layer_forward keeps one workspace per stream it
 *     is called on, and moe_layer_forward_ws runs on a workspace the caller
 *     owns, so calls on different streams (or workspaces) share no scratch.
 *     Host threads may call concurrently; moe_layer_set_routing and
 *     moe_layer_set_mode apply to calls made after they return.
 *   - Inside a forward call on the few-tokens or MFMA path, a layer with a
 *     shared expert encodes x and runs the shared expert on a stream the
 *     context owns, which waits for `stream` (an event) before it starts;
 *     `stream` waits for x's encoding before its first expert kernel and
 *     for the shared expert before the combine: the call stays ordered on
 *     `stream` as a whole.  Calls on a
 *     stream that is being captured into a graph, and
 *     moe_layer_forward_noalloc, keep every launch on `stream`.
 */
#ifndef MOE_HIP_H
#define MOE_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes. */
#define MOE_OK 0
#define MOE_EINVAL (-1)   /* bad argument, shape or format */
#define MOE_ENOMEM (-2)   /* device or host allocation failed */
#define MOE_EHIP (-3)     /* a HIP runtime call failed */
#define MOE_EUNSUP (-4)   /* valid for the reference, not supported here */

/* Storage formats, numbered as GGUF numbers them.  Replaces quant::Dt
 * (src/quant.rs:19-37); Q4_0/Q5_0/Q8_0 are byte-identical to the engine's
 * Dt::Q4/Q5/Q8 (src/gguf.rs:165-173). */
#define MOE_DT_F32 0
#define MOE_DT_F16 1
#define MOE_DT_Q4_0 2
#define MOE_DT_Q5_0 6
#define MOE_DT_Q8_0 8
#define MOE_DT_BF16 30
/* The reference's own 6-bit format (Dt::Q6, 26 bytes per 32 values), which
 * a .moe file may hold; listed by the container reader, read by no kernel. */
#define MOE_DT_Q6_REF (-2)

/* Gate kinds (Spec::sigmoid, src/spec.rs:305-306). */
#define MOE_GATE_SOFTMAX 0
#define MOE_GATE_SIGMOID 1

typedef struct moe_ctx moe_ctx;
typedef struct moe_layer moe_layer;

/* A 2-D row-major weight view inside an uploaded region.  Replaces quant::QT
 * (src/quant.rs:97-129) as produced by Store::view (src/store.rs:303-315):
 * `offset` is the byte offset of the view's first row inside the region,
 * rows are Dt::row_bytes(cols) apart (src/quant.rs:68-83).  dt < 0 means
 * "absent" for optional tensors. */
typedef struct moe_tensor {
    int32_t dt;
    int32_t rows;
    int32_t cols;
    int32_t _reserved;
    uint64_t region;
    uint64_t offset;
} moe_tensor;

/* One routed layer: the fields of Ffn::Moe (src/model.rs:68-71) plus the
 * Spec routing scalars it reads (src/spec.rs:199-207). */
typedef struct moe_layer_desc {
    int32_t hidden;        /* H */
    int32_t n_experts;     /* E */
    int32_t top_k;         /* Spec::top_k */
    int32_t gate;          /* MOE_GATE_* */
    int32_t norm_topk;     /* Spec::norm_topk */
    int32_t n_group;       /* Spec::n_group (1 = no group limit) */
    int32_t topk_group;    /* Spec::topk_group */
    float routed_scale;    /* Spec::routed_scale */
    moe_tensor router;     /* F32 [E, H]   (mlp.gate.weight) */
    moe_tensor e_bias;     /* F32 [1, E] or dt<0 (mlp.gate.e_score_correction_bias) */
    const moe_tensor *experts; /* 3*E views: expert e at [3e+0]=gate [I,H], [3e+1]=up [I,H], [3e+2]=down [H,I] */
    moe_tensor shared[3];  /* gate, up, down of the shared expert, or dt<0 */
    moe_tensor shared_gate;/* F32 [1, H] or dt<0 (mlp.shared_expert_gate.weight) */
} moe_layer_desc;

/* Router interventions for one layer.  Replaces model::Routing
 * (src/model.rs:238-280) as applied at src/model.rs:846-888. */
typedef struct moe_routing {
    const int32_t *disabled; /* expert ids this layer may not select (host memory) */
    int32_t n_disabled;
    const int32_t *forced;   /* expert ids always selected, in order (host memory) */
    int32_t n_forced;
    float temp;              /* divides the logits when > 0 */
    int32_t top_k;           /* overrides Spec::top_k when > 0 */
} moe_routing;

/* One routing decision: Route::experts entries (src/model.rs:84-91). */
typedef struct moe_route {
    uint32_t expert;
    float weight;
} moe_route;

/* ------------------------------------------------------------------ setup */

/* Open a context on HIP device `device`, with one non-blocking stream of
 * default priority for the layers' shared experts.  Replaces Model::load's
 * ownership of the Store (src/model.rs:336-341). */
int moe_ctx_create(int device, moe_ctx **out);
void moe_ctx_destroy(moe_ctx *ctx);

/* Copy `bytes` of host memory (e.g. an mmap'd checkpoint range) into a new
 * 256-byte-aligned device region and return its handle.  Replaces
 * Store::open's mmap (src/store.rs:72-77, 126-136): byte offsets inside the
 * region are preserved, so views address it exactly as Store::view does. */
int moe_upload(moe_ctx *ctx, const void *host, uint64_t bytes, uint64_t *region_out);

/* Device address of a region (for callers that fill regions themselves). */
int moe_region_ptr(moe_ctx *ctx, uint64_t region, void **dev_out);

/* Build a layer over uploaded views.  Replaces the per-layer binding in
 * Model::load_with (src/model.rs:396-441).  Validates formats, shapes and
 * that every view lies inside its region (Rec::fits_in, src/store.rs:44-46). */
int moe_layer_create(moe_ctx *ctx, const moe_layer_desc *desc, moe_layer **out);
void moe_layer_destroy(moe_layer *layer);

/* Install router interventions (NULL clears them).  Replaces setting
 * Model::routing for one layer (src/model.rs:238-280).  The interventions
 * travel by value in each call's kernel arguments: calls already queued keep
 * the routing they were made with. */
int moe_layer_set_routing(moe_layer *layer, const moe_routing *routing);

/* Allocate the workspace moe_layer_forward uses on `stream` for up to
 * `max_t` tokens (at the current top_k or the layer's own, whichever is
 * larger).  After a reservation no forward call allocates on that stream,
 * and a call with more tokens (or, after set_routing, more experts per token)
 * than reserved fails with MOE_EINVAL.  Without one, moe_layer_forward
 * allocates a stream's workspace on its first call there and grows it when
 * t grows, by at least half its size each time; an outgrown workspace is
 * freed once the work queued before the growth has finished (queried at a
 * later growth, never waited for) or by moe_layer_destroy.  No
 * counterpart in the reference, which allocates scratch per call
 * (src/model.rs:900-935). */
int moe_layer_reserve_stream(moe_layer *layer, int32_t max_t, void *stream);
/* moe_layer_reserve_stream on the null stream. */
int moe_layer_reserve(moe_layer *layer, int32_t max_t);

/* Drop the workspace moe_layer_forward keeps for `stream`: it is freed once
 * the work already queued on the stream has finished (checked without
 * waiting at later workspace growth, and at moe_layer_destroy).  Call it
 * before destroying a stream whose handle value a new stream may reuse:
 * workspaces are keyed by the handle.  No counterpart in the reference. */
int moe_layer_release_stream(moe_layer *layer, void *stream);

/* Bytes of a caller-owned workspace for moe_layer_forward_ws over up to
 * `max_t` tokens at the layer's current top_k. */
int moe_layer_workspace_size(const moe_layer *layer, int32_t max_t, uint64_t *bytes);

/* Kernel path: 0 = automatic (one-token integer-dot kernels at t = 1,
 * few-tokens integer-dot kernels while the hit experts average at most 3
 * tokens (1.5 for rows wider than 4096), MFMA grouped GEMM beyond, register
 * GEMV for shapes the MFMA kernel does not take, exact kernels for shapes
 * none fits), 1 = exact kernels
 * (bit-identical to the CPU path, slow), 2 = GEMV, 3 = MFMA, 4 = one-token
 * kernels at t = 1 and GEMV otherwise, 5 = few-tokens integer-dot kernels
 * (up to 256 tokens), 6 = MFMA grouped GEMM with the weights streamed
 * through a deep LDS ring (eight waves per tile, same arithmetic as 3;
 * shapes it does not take fall back as 3 does).  Every path computes in f32 precision: the GEMV and
 * exact kernels in f32 arithmetic, the integer-dot kernels on activations
 * held as three int8 levels (2^-24 of each 32-value block's range), the
 * MFMA kernels on two-piece f16 operands (exact weights, 22-bit
 * activations) accumulated in f32.  No counterpart in the reference, which
 * has one CPU path. */
int moe_layer_set_mode(moe_layer *layer, int mode);

/* Keep (enable != 0) or drop a second, tiled copy of the layer's expert
 * matrices on the device: each 32-row region's 64-value steps contiguous,
 * each row's step with the bytes one MFMA lane needs side by side (Q4_0,
 * Q5_0 and Q8_0 with K % 64 == 0; otherwise MOE_EUNSUP).  It costs the
 * experts' bytes again (plus row padding to 32) and makes calls whose
 * experts average at most ~20 tokens (t > 1) stream it through registers
 * at about twice the rate of the row-major views; mode 6 uses it for its
 * 32-token tiles.  Waits for the device; not to be called while another
 * thread runs a forward on this layer.  No counterpart in the reference,
 * which keeps one row-major copy. */
int moe_layer_set_tiled(moe_layer *layer, int enable);

/* Experts each token is routed to (min(top_k, E)) under the current routing. */
int moe_layer_k(const moe_layer *layer);

/* ---------------------------------------------------------------- forward */

/* The routed layer over `t` tokens.  Replaces Model::feed_forward's Ffn::Moe
 * arm (src/model.rs:841-971) and, when `residual` is given, trunk's residual
 * add that follows it (src/model.rs:680-683).
 *   x        device f32 [t, H]  layer input (post-norm activations)
 *   out      device f32 [t, H]  overwritten with the layer output (delta)
 *   residual device f32 [t, H]  or NULL; if given, residual += out
 *   routes   device [t, k]      or NULL; routing table strongest first
 *                               (Route.experts, src/model.rs:943-950)
 *   hits     device u32 [E+1]   or NULL; hits[0] = n, hits[1..n] = experts
 *                               with >= 1 token, ascending (State::prev,
 *                               src/model.rs:951)
 *   prev     device u32 [E+1]   or NULL; the previous call's `hits`, used for
 *                               the reuse counter (src/model.rs:913-916)
 *   stats    device u64 [4]     or NULL; += routed, reused, expert_bytes and
 *                               tokens with an exact rank tie in the selected
 *                               prefix (Stats, src/model.rs:116-126)
 */
int moe_layer_forward(moe_layer *layer, const float *x, int32_t t, float *out, float *residual, moe_route *routes,
                      uint32_t *hits, const uint32_t *prev, uint64_t *stats, void *stream);

/* moe_layer_forward on a caller-owned workspace: `workspace` is device
 * memory of `workspace_bytes` (>= moe_layer_workspace_size for t tokens),
 * 256-byte aligned, zero-filled before its first use (every call leaves the
 * counters it keeps there at zero again).  Allocates nothing.  Calls on
 * different workspaces may run concurrently on any streams; calls that
 * share a workspace must be ordered (one stream).  Replaces the same
 * feed_forward arm as moe_layer_forward (src/model.rs:836-971), whose
 * State is per sequence. */
int moe_layer_forward_ws(moe_layer *layer, const float *x, int32_t t, float *out, float *residual,
                         moe_route *routes, uint32_t *hits, const uint32_t *prev, uint64_t *stats, void *workspace,
                         uint64_t workspace_bytes, void *stream);

/* moe_layer_forward on a fixed 64 MiB device array that the library's code
 * object carries (one per device, looked up once per device on the first
 * call there): allocates nothing, ever.  No counterpart in the reference;
 * for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc).  A call
 * whose workspace would exceed the array (moe_layer_workspace_size) fails
 * with MOE_EINVAL; calls that overlap on one device share the array and race,
 * so order them on one stream.  Stage timing is not recorded. */
int moe_layer_forward_noalloc(moe_layer *layer, const float *x, int32_t t, float *out, float *residual,
                              moe_route *routes, uint32_t *hits, const uint32_t *prev, uint64_t *stats,
                              void *stream);

/* Router logits and gating only: routes [t, k] for x [t, H], as
 * src/model.rs:844-898 computes them.  `logits` (device f32 [t, E]) may be
 * NULL; if given it receives the router logits after the temperature. */
int moe_layer_route(moe_layer *layer, const float *x, int32_t t, moe_route *routes, float *logits, void *stream);

/* Stage timing (no counterpart in the reference).  While enabled, forward
 * records HIP events around each of its stages on the call's stream:
 * 0 router, 1 gating, 2 dispatch, 3 expert gate/up, 4 expert down,
 * 5 combine, 6 activation encoding (f16 pieces or int8 levels of x and h).
 * moe_layer_stage_times synchronises on the recorded events and adds each
 * stage's accumulated milliseconds and launch count into ms[7], n[7], then
 * resets the accumulators. */
#define MOE_STAGES 7
int moe_layer_profile(moe_layer *layer, int enable);
int moe_layer_stage_times(moe_layer *layer, double *ms, uint64_t *n);

const char *moe_last_error(void);

/* Test hook: y[i] = exp(x[i]) computed on the device by the gates' exp (a
 * port of glibc's expf), for checking it against the host libm.  x and y are
 * device f32 [n].  No counterpart in the reference. */
int moe_debug_expf(const float *x, float *y, uint64_t n, void *stream);

/* Test hook: which one-token gate/up kernel the forward uses, for every
 * layer of the process: 0 the automatic choice, 1 the strided kernel with
 * its separate encoding of h, 2 the unit-aligned kernel that encodes h
 * itself.  Returns the previous choice (>= 0) or MOE_EINVAL.  Both give the
 * same bits.  No counterpart in the reference. */
int moe_debug_decode_kernel(int32_t choice);

/* Test hook: which MFMA kernels the fast paths use, for every layer and
 * projection of the process: 0 the two-pass kernels (weight codes times
 * the activations' two f16 pieces, the block scale applied to each block's
 * f32 sum), 1 the three-pass kernels (both operands in two f16 pieces).
 * Returns the previous choice (>= 0) or MOE_EINVAL.  No counterpart in the
 * reference. */
int moe_debug_mfma_kernel(int32_t choice);

/* ------------------------------------------------ the model around the layer
 * The rest of the reference's forward (src/model.rs:646-834) as device
 * operations, so that a whole decoder runs with its routed layers on the
 * kernels above.  All tensors are device f32 unless stated; `stream` as
 * above.  These compute in f32 and reduce in their own order: results agree
 * with the CPU path to f32 rounding. */

typedef struct moe_linear moe_linear;

/* A plain projection y = W x over an uploaded view W [N, K] in any format of
 * this library (F32, Q4_0, Q5_0, Q8_0).  Replaces quant::matmul
 * (src/quant.rs:482-506) for the attention projections, the dense layers'
 * matrices and lm_head (src/model.rs:641, 704-706, 742-771, 833), on the
 * expert kernels: the f32 GEMV for up to 8 tokens, the MFMA kernel (two-piece
 * f16 operands, f32 accumulation) beyond, the exact kernel (the reference's
 * dot, bit for bit) for formats and widths those do not take. */
int moe_linear_create(moe_ctx *ctx, const moe_tensor *w, moe_linear **out);
void moe_linear_destroy(moe_linear *linear);
/* Bytes of workspace moe_linear_forward needs for up to max_t tokens. */
int moe_linear_workspace_size(const moe_linear *linear, int32_t max_t, uint64_t *bytes);
/* y [t, N] = x [t, K] W^T; residual (or NULL) += y.  `workspace`: device,
 * 256-byte aligned, moe_linear_workspace_size bytes (ordered on one stream). */
int moe_linear_forward(moe_linear *linear, const float *x, int32_t t, float *y, float *residual, void *workspace,
                       uint64_t workspace_bytes, void *stream);

/* x[i] = the dequantised row tokens[i] % rows of a table stored in `dt`
 * (trunk's embedding lookup, src/model.rs:669-671).  table: device bytes of
 * rows x Dt::row_bytes(cols); tokens: device int32 [t]. */
int moe_embed_rows(const void *table, int32_t dt, int32_t rows, int32_t cols, const int32_t *tokens, int32_t t,
                   float *x, void *stream);

/* rmsnorm (src/model.rs:211-216) of `rows` rows of n values, x_stride and
 * out_stride floats apart, weight w [n]. */
int moe_rmsnorm(const float *x, int64_t x_stride, const float *w, int32_t rows, int32_t n, float eps, float *out,
                int64_t out_stride, void *stream);

/* rope (src/model.rs:324-333) in place: for each row r (row_stride floats
 * apart) and head h < heads (head_stride floats apart), the dim values from
 * `offset` rotate pairwise (i, i + dim/2) by pos[r] * inv_freq[i].
 * pos: device int32 [rows]; inv_freq: device f32 [n_inv]. */
int moe_rope(float *x, int32_t rows, int64_t row_stride, int32_t heads, int32_t head_stride, int32_t offset,
             int32_t dim, const int32_t *pos, const float *inv_freq, int32_t n_inv, void *stream);

/* Rope::inv_freqs (src/spec.rs:89-145) on the host into out[head_dim / 2]:
 * kind 0 none, 1 linear, 2 dynamic (NTK), 3 YaRN, 4 Llama 3. */
int moe_rope_inv_freqs(int32_t kind, float theta, float factor, uint64_t original_ctx, float low_freq_factor,
                       float high_freq_factor, float beta_fast, float beta_slow, int32_t head_dim, float *out);

/* x[i] += bias[i % bias_len] over `total` values (src/model.rs:707-713). */
int moe_add_bias(float *x, uint64_t total, const float *bias, int32_t bias_len, void *stream);

/* dst row dst_rows[r] (dst_stride floats apart) = src row r (n values,
 * src_stride apart): the KV-cache write (src/model.rs:732-733).
 * dst_rows: device int64 [rows]. */
int moe_scatter_rows(const float *src, int32_t rows, int32_t n, int64_t src_stride, float *dst, int64_t dst_stride,
                     const int64_t *dst_rows, void *stream);

/* MLA's cache rows (src/model.rs:773-787): for row r and head h, key
 * [kv nope part, c's rope part (k_pe, already rotated)] and value kv's value
 * part, written at cache row dst_rows[r].  kv [rows, heads * (qk_nope +
 * v_head)], c [rows, >= kv_lora + qk_rope] c_stride apart. */
int moe_mla_kv_store(const float *kv, const float *c, int64_t c_stride, int32_t kv_lora, int32_t rows,
                     int32_t heads, int32_t qk_nope, int32_t qk_rope, int32_t v_head, float *kcache, float *vcache,
                     const int64_t *dst_rows, void *stream);

/* Causal attention (src/model.rs:790-831): row r of q (heads x qd values,
 * q_stride apart) belongs to sequence seq[r] at position pos[r] and attends
 * to cache positions [lo, pos[r]] of that sequence (lo = pos + 1 - window
 * for window > 0, else 0), head h reading kv head h / (heads / n_kv) when
 * heads / n_kv > 1, else kv head min(h, n_kv - 1).
 * Cache layout: [sequence][ctx][n_kv * qd] keys, [sequence][ctx][n_kv * vd]
 * values.  out row r: heads x vd values.  max_pos bounds every pos[r]. */
int moe_attention(const float *q, int64_t q_stride, int32_t rows, int32_t heads, int32_t n_kv, int32_t qd,
                  int32_t vd, float scale, const float *kcache, const float *vcache, int64_t ctx, const int32_t *seq,
                  const int32_t *pos, int32_t max_pos, int32_t window, float *out, int64_t out_stride, void *stream);

/* out[r] = the first index of row r's maximum (greedy sampling,
 * src/sample.rs:87-95).  x [rows, n]; out: device int32 [rows]. */
int moe_argmax(const float *x, int32_t rows, int32_t n, int32_t *out, void *stream);

/* --------------------------------------------------- checkpoint containers */

/* One tensor of a single-file checkpoint: Store's Rec (src/store.rs:25-47).
 * `offset` is the byte offset of the first row from the start of the file;
 * a 3-D expert stack is `slabs` x `rows` rows of width `cols`, rows
 * Dt::row_bytes(cols) apart (src/quant.rs:68-83).  `dt` is MOE_DT_* (GGUF's
 * numbering, so other GGUF types keep their ggml number), `bytes` the size
 * (0 for a type whose row size this library does not know). */
typedef struct moe_rec {
    const char *name;      /* owned by the container */
    int32_t dt;
    int32_t _reserved;
    uint64_t slabs, rows, cols;
    uint64_t offset;
    uint64_t bytes;
} moe_rec;

typedef struct moe_container moe_container;

/* Parse a packed `.moe` file (src/store.rs:228-279) or a GGUF v2/v3 file
 * (src/gguf.rs:206-276) held in caller-owned memory (typically an mmap that
 * outlives the container).  Every length in the header is checked against
 * `len`: a corrupt or truncated file is MOE_EINVAL, never an out-of-bounds
 * read.  Replaces Store::open for single-file checkpoints. */
int moe_container_open(const void *bytes, uint64_t len, moe_container **out);
void moe_container_close(moe_container *c);
/* 1 = .moe, 2 = GGUF. */
int moe_container_kind(const moe_container *c);
int64_t moe_container_count(const moe_container *c);
int moe_container_rec(const moe_container *c, int64_t i, moe_rec *out);
/* Store::shape / Store::has by name (src/store.rs:293-301, 317-319). */
int moe_container_find(const moe_container *c, const char *name, moe_rec *out);
/* A .moe header's "config" object as JSON text (Store::config), or NULL. */
const char *moe_container_config(const moe_container *c);

/* The Hugging Face name of a GGUF tensor (gguf::rename, src/gguf.rs:435-487)
 * into out[cap]; returns 1 (and leaves out alone) for tensors with no
 * counterpart, such as rope frequency tables. */
int moe_gguf_rename(const char *name, char *out, uint64_t cap);

/* Upload n tensors of a host buffer (byte ranges [offsets[i], offsets[i] +
 * lengths[i]) of host[host_len]) into one new device region, each starting
 * on a 256-byte boundary; dev_offsets_out[i] receives tensor i's offset in
 * the region.  Rows keep their offsets relative to their tensor, so a view
 * of a tensor addresses the region as Store::view addresses the file; the
 * kernels' wide loads get aligned rows even where the file packs tensors
 * back to back (.moe payloads are unpadded, src/store.rs:439-441). */
int moe_upload_tensors(moe_ctx *ctx, const void *host, uint64_t host_len, const uint64_t *offsets,
                       const uint64_t *lengths, int64_t n, uint64_t *dev_offsets_out, uint64_t *region_out);

/* ------------------------------------------------------- host utilities */

/* Dt::row_bytes (src/quant.rs:68-83); 0 for an unknown format. */
uint64_t moe_row_bytes(int32_t dt, uint64_t cols);

/* quant::quantize over `rows` rows (src/quant.rs:304-365): F32, F16, Q8_0,
 * Q4_0, Q5_0.  cols must fit the format (Dt::fits, src/quant.rs:86-92). */
int moe_quantize_rows(int32_t dt, const float *src, uint64_t rows, uint64_t cols, uint8_t *dst);

/* quant::dequant over `rows` rows (src/quant.rs:177-227). */
int moe_dequant_rows(int32_t dt, const uint8_t *src, uint64_t rows, uint64_t cols, float *dst);

/* Seeded synthetic data (no counterpart in the reference, which has no normal
 * generator): element i of stream (seed, stream) is mean + std*z_i, z from
 * Box-Muller over splitmix64 uniforms, computed in double then rounded to
 * float.  Multithreaded, deterministic. */
int moe_synth_normal(uint64_t seed, uint64_t stream, uint64_t n, double mean, double std, float *out);

/* The same values, quantised row by row as quantize would store them, without
 * materialising the f32 tensor.  dst holds rows * row_bytes(dt, cols). */
int moe_synth_quantized(uint64_t seed, uint64_t stream, int32_t dt, uint64_t rows, uint64_t cols, double mean,
                        double std, uint8_t *dst);

#ifdef __cplusplus
}
#endif
#endif /* MOE_HIP_H */
