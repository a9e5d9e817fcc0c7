/*
 * moe_ffn.h -- C ABI of the MI355X-native MoE expert-FFN hot path (gfx950, HIP).
 *
 * Drop-in for the Vulkan MoE path of herlangga72/moe-680m.  Every entry point below names
 * the reference interface it replaces (path:line in the reference tree).  The reference
 * binds that path from Rust (src/inference.rs, src/router.rs); the matching Rust
 * `extern "C"` block is in INTEGRATION.md.
 *
 * Conventions
 *   - All tensor pointers are DEVICE pointers; the caller owns every buffer.
 *   - Calls are asynchronous on the given HIP stream (`void*` = hipStream_t, NULL = the
 *     legacy default stream); nothing in a hot call synchronises the host or allocates.
 *   - Every function returns a moe_status; on failure moe_last_error() returns a message
 *     (thread-local).  Nothing throws or aborts across this boundary.
 *   - One context per stream/thread at a time; contexts hold no locks.
 *   - Layout: activations f32 row-major [M][hidden]; weights GGML IQ4_XS (136-byte
 *     super-blocks of 256 weights), row-major [out][in] (rows are outputs, K contiguous).
 *     Weight bases and strides must be multiples of 16 bytes.
 *   - Routing: ids u16 [M][9], w f32 [M][9].  Slots 0..7 hold the routed experts in
 *     descending logit order, slot 8 the shared expert with id = n_experts and weight 1.
 */
#ifndef MOE_FFN_H
#define MOE_FFN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct moe_ctx moe_ctx;

typedef enum {
    MOE_OK = 0,
    MOE_EINVAL = 1,       /* bad argument (null pointer, size, alignment, layer index) */
    MOE_ENOMEM = 2,       /* device allocation failed at create time */
    MOE_EHIP = 3,         /* a HIP runtime call failed */
    MOE_EUNSUPPORTED = 4, /* shape not compiled into this library */
    MOE_EDEVICE = 5       /* a kernel flagged invalid device-side input (see moe_device_flags) */
} moe_status;

/* Weight convention of the 8 routed slots.
 *   MOE_W_REF:    w = softmax probability (not renormalised) and every expert's output,
 *                 the shared one included, is scaled by 1/9 -- src/router.rs:37-48,
 *                 src/inference.rs:720,750.
 *   MOE_W_RENORM: w renormalised over the 8 selected experts, scale 1. */
typedef enum { MOE_W_REF = 0, MOE_W_RENORM = 1 } moe_wmode;

enum { MOE_TOPK = 8, MOE_SLOTS = 9, MOE_DECODE_MAX_M = 8, MOE_MAX_EXPERTS = 256 };

/* moe_ffn flags (and moe_decode_stack's) */
enum {
    MOE_FFN_ACCUMULATE = 1,  /* y += out (fused residual); otherwise y = out */
    MOE_FFN_RMSNORM = 2,     /* FFN input is x / sqrt(mean(x^2) + 1e-6) (unit gain) */
    MOE_STACK_ROUTE_GEMV = 4 /* moe_decode_stack only: route every layer from its own input
                                with the router bound by moe_bind_router (no logits) */
};

/* Device-side input flags (sticky per context, read by moe_device_flags). */
enum {
    MOE_DEVFLAG_BAD_ID = 1,   /* an expert id > n_experts was seen; its slot was dropped */
    MOE_DEVFLAG_DUP_ID = 2,   /* a token named one expert in two slots; the later was dropped */
    MOE_DEVFLAG_TIMEOUT = 4   /* moe_decode_stack: a bounded wait expired; its output is invalid */
};

typedef struct {
    int hidden;     /* 2048 for moe-680m (also 512 is compiled, for small tests) */
    int inter;      /* 512 for moe-680m (also 256 is compiled) */
    int n_experts;  /* routed experts, 8..256 (256 for moe-680m); shared id = n_experts */
    int n_layers;   /* weight tables to hold (40 for moe-680m) */
    int m_max;      /* largest M any call will pass (<= 65535); sizes the workspaces */
    moe_wmode wmode;
} moe_config;

/* One layer's experts.  Routed expert e: W1 at w1 + e*w1_stride, W3 at w3 + e*w3_stride,
 * W2 at w2 + e*w2_stride.  W1, W3: [inter][hidden]; W2: [hidden][inter].
 * Replaces LayerWeights::{expert_w1,expert_w3,expert_w2,shared_w1,shared_w3,shared_w2}
 * (src/memory.rs:201-291, indexed layer*256+e at src/inference.rs:730,759). */
typedef struct {
    const void *w1, *w3, *w2;
    size_t w1_stride, w3_stride, w2_stride;
    const void *shared_w1, *shared_w3, *shared_w2;
} moe_layer_weights;

/* Create a context on HIP device `device`: validates the shape, allocates every
 * workspace for m_max tokens and the one device copy of the weights that moe_bind_layer
 * fills (nothing is allocated later): n_layers x (E+1) x 3 matrices in the library's split
 * layout, which every kernel family reads.
 * Replaces the MoE slice of InferenceEngine::new (src/inference.rs:85-126) and the
 * scratch / routing regions of ArenaLayout::compute (src/memory.rs:32-96). */
moe_status moe_create(int device, const moe_config *cfg, moe_ctx **out);
moe_status moe_destroy(moe_ctx *ctx);

/* Copy one layer's weights (device pointers, read only during this call) into the context's
 * split layout (same bytes, qs and headers of each super-block apart).  Synchronises the
 * device: the caller's buffers may be freed when it returns.  Rebinding a layer replaces its
 * copy.
 * Replaces LayerWeights::from_registry (src/memory.rs:227-291). */
moe_status moe_bind_layer(moe_ctx *ctx, int layer, const moe_layer_weights *lw);

/* Bind layer `layer`'s router gate matrix for moe_decode_stack's MOE_STACK_ROUTE_GEMV form:
 * wg [n_experts][hidden] of element type wg_type (MOE_WG_IQ4_XS, MOE_WG_F32, MOE_WG_F16 --
 * declared below), rows = experts, 16-byte aligned device memory.  The library keeps the
 * pointer, not a copy: the matrix must stay valid while bound.  wg = NULL unbinds.
 * Replaces the ffn_gate entry of LayerWeights::from_registry (src/memory.rs:236-262), which
 * the Router dispatch reads (src/inference.rs:598-605). */
moe_status moe_bind_router(moe_ctx *ctx, int layer, const void *wg, int wg_type);

/* Softmax + top-8 per token: logits f32 [M][n_experts] -> ids u16 [M][9], w f32 [M][9].
 * Ties go to the lower index; NaN logits never win and count as -inf in the softmax.
 * Replaces shaders/router_topk.comp (dispatch src/inference.rs:608-616) and
 * router::route_single / route_cpu (src/router.rs:13-51) as used by do_route
 * (src/inference.rs:622-659). */
moe_status moe_router_topk(moe_ctx *ctx, const float *logits, int M, uint16_t *ids, float *w,
                           void *stream);

/* Router gate GEMV fused with the top-8: logits[t][e] = sum_k xin[t][k] * Wg[e][k], xin = x_t
 * or, with flags = MOE_FFN_RMSNORM, RMSNorm(x_t) (eps 1e-6, no gain); then ids/w exactly as
 * moe_router_topk computes them from those logits (a second launch).  wg: IQ4_XS
 * [n_experts][hidden] in the GGML layout (rows = experts, 16-byte
 * aligned device memory, read in place -- no binding; other element types:
 * moe_router_gemv_topk_typed);
 * x f32 [M][hidden]; logits f32 [M][n_experts] or NULL (then M <= m_max and the context's
 * workspace holds them); ids u16 / w f32 [M][9], or both NULL for logits only.  f32
 * arithmetic throughout (exact weights).  Replaces the Router GEMV dispatch
 * (shaders/router.comp:21-61 at src/inference.rs:598-605) and, with ids/w, the RouterTopk
 * dispatch and do_route (src/inference.rs:608-659). */
moe_status moe_router_gemv_topk(moe_ctx *ctx, const void *wg, const float *x, int M, int flags,
                                float *logits, uint16_t *ids, float *w, void *stream);

/* Element types of the router gate matrix, by their GGML type ids (the ids a GGUF file's
 * tensor table gives ffn_gate_inp): llama.cpp's quantizer keeps that tensor F32 or F16. */
enum { MOE_WG_F32 = 0, MOE_WG_F16 = 1, MOE_WG_IQ4_XS = 23 };

/* moe_router_gemv_topk with the gate matrix's element type given: wg [n_experts][hidden] as
 * IQ4_XS super-blocks (MOE_WG_IQ4_XS), f32 (MOE_WG_F32) or f16 (MOE_WG_F16), row-major, rows
 * = experts, 16-byte aligned device memory, read in place.  f32 arithmetic (f16 weights
 * converted exactly).  With ids/w the top-8 is a second launch.  Replaces the Router GEMV dispatch
 * (shaders/router.comp:21-61 at src/inference.rs:598-605) on the weight the loader found
 * (src/memory.rs:236-262 binds blk.L.ffn_gate) and, with ids/w, the RouterTopk dispatch and
 * do_route (src/inference.rs:608-659). */
moe_status moe_router_gemv_topk_typed(moe_ctx *ctx, const void *wg, int wg_type, const float *x, int M,
                                      int flags, float *logits, uint16_t *ids, float *w, void *stream);

/* Prefix-sum expert bucket fill over n_experts+1 buckets (bucket n_experts = shared):
 * ranges u32 [n_experts+2], sorted_tok u16 [9M], sorted_w f32 [9M]; tokens ascend inside
 * a bucket.  Replaces router::build_expert_batches (src/router.rs:55-97) and the upload
 * of its output (src/inference.rs:684-699). */
moe_status moe_bucket_fill(moe_ctx *ctx, const uint16_t *ids, const float *w, int M,
                           uint32_t *ranges, uint16_t *sorted_tok, float *sorted_w, void *stream);

/* The expert FFN of one layer for M tokens and the weighted combine:
 *   out_t = c * sum_{s<9} w[t][s] * W2_e (silu(W1_e xin_t) * (W3_e xin_t)),  e = ids[t][s]
 *   y_t   = (flags & ACCUMULATE ? y_t : 0) + out_t
 * c = 1/9 (MOE_W_REF) or 1 (MOE_W_RENORM).  x and y may be the same buffer.  A slot whose
 * id exceeds n_experts, or repeats an id of an earlier slot of its token, is dropped
 * (MOE_DEVFLAG_BAD_ID / MOE_DEVFLAG_DUP_ID), for every M.
 * M <= 8 runs the decode path, IQ4_XS GEMV launches (activations -- and, at M >= 2, the
 * down product's h -- as two int8 planes per 32-element chunk, f32 accumulation; each
 * selected expert's weights read once however many tokens chose it); larger M runs bucket fill + grouped f16-MFMA GEMMs (f32
 * accumulate) + combine.  Replaces record_and_submit_moe (src/inference.rs:663-766): shaders
 * w1_w3_fused(_m1).comp, silu_mult.comp, w2(_scatter)(_m1).comp, moe_combine.comp. */
moe_status moe_ffn(moe_ctx *ctx, int layer, const float *x, const uint16_t *ids, const float *w,
                   int M, float *y, int flags, void *stream);

/* Router and expert FFN of one layer in one call: (ids, w) = top8(softmax(logits)) exactly
 * as moe_router_topk computes them (written to ids/w, [M][9]), then moe_ffn with them.  For
 * M <= 8 the routing runs inside the decode launches (no separate router launch).
 * Replaces the RouterTopk dispatch (src/inference.rs:608-616), do_route's readback
 * (src/inference.rs:622-659) and record_and_submit_moe (src/inference.rs:663-766) of one
 * layer. */
moe_status moe_ffn_route(moe_ctx *ctx, int layer, const float *x, const float *logits, int M,
                         float *y, uint16_t *ids, float *w, int flags, void *stream);

/* moe_ffn for M <= MOE_DECODE_MAX_M whose h scratch is a static device array of the library
 * (191,744 bytes per GPU, held until the process ends) instead of the context's workspace:
 * nothing in this call allocates, frees or calls an allocating library routine.  No
 * counterpart in the reference; it is for callers that cannot allocate device memory
 * (work under graph capture, tight serving loops, harnesses that forbid allocation).
 * Refuses M > MOE_DECODE_MAX_M and inter > 512 (MOE_EINVAL / MOE_EUNSUPPORTED).  Every call
 * on a GPU shares that GPU's array: calls that overlap on one GPU (two streams) race. */
moe_status moe_ffn_noalloc(moe_ctx *ctx, int layer, const float *x, const uint16_t *ids, const float *w,
                           int M, float *y, int flags, void *stream);

/* One token (M = 1) through n_layers consecutive MoE layers in one persistent launch (the
 * routing of every layer runs inside it; nothing else is launched):
 *   for l in layer0 .. layer0+n_layers-1:
 *       xin = RMSNorm(x) if asked, else x
 *       (ids_l, w_l) = top8(softmax(logits[l - layer0]))      (as moe_router_topk)
 *          or, with MOE_STACK_ROUTE_GEMV, top8(softmax(Wg_l xin)), Wg_l the router bound
 *          to layer l (as moe_router_gemv_topk_typed, with xin read as the two int8 planes
 *          per 32 elements the expert products read; logits within 1 ulp of f32 sums)
 *       x = x + c * sum_{s<9} w_l[s] * FFN_{ids_l[s]}(xin)
 *   y = x  (y may be the same buffer as x)
 * logits f32 [n_layers][n_experts] (NULL with MOE_STACK_ROUTE_GEMV); ids u16 / w f32
 * [n_layers][9] receive the routing (both may be NULL).  flags: MOE_FFN_RMSNORM,
 * MOE_STACK_ROUTE_GEMV (the residual is always added).
 * Needs n_experts <= 256 and every workgroup of the launch resident at once (one per CU;
 * checked at moe_create), hidden/8 workgroups spread evenly over the device's 8 XCDs.
 * Every wait inside the launch is bounded: one that expires sets MOE_DEVFLAG_TIMEOUT, every
 * workgroup then stops publishing and leaves, and y is left unwritten -- it is written only
 * after every row of the last layer is complete -- so an x that y aliases keeps its value.
 * Check the flag with moe_device_flags or, without a host sync, moe_device_flags_async; both
 * also reset the stack's internal state when they find it, and until then later launches may
 * fail the same way (never with a silently wrong y).
 * Replaces, for the MoE path of one decode token, the per-layer sequence
 * record_and_submit_layer's RouterTopk dispatch -> do_route -> record_and_submit_moe of
 * InferenceEngine::forward_single (src/inference.rs:296-301, 608-616, 622-766) -- with
 * MOE_STACK_ROUTE_GEMV also its Router dispatch (src/inference.rs:598-605). */
moe_status moe_decode_stack(moe_ctx *ctx, int layer0, int n_layers, const float *x,
                            const float *logits, float *y, uint16_t *ids, float *w, int flags,
                            void *stream);

/* IQ4_XS decode of n_superblocks blocks into f32 [256*n] (test hook for the codec).
 * Replaces dequant_iq4_xs (shaders/common.glsl:61-86) with the GGML 136-byte format. */
moe_status moe_dequant_iq4xs(const void *blocks, size_t n_superblocks, float *out, void *stream);

/* Synchronise the context's last stream and return (then clear) the sticky device flags.
 * No reference counterpart: the reference panics instead (src/router.rs:41). */
moe_status moe_device_flags(moe_ctx *ctx, void *stream, uint32_t *flags);

/* Stream-ordered variant for callers that cannot block (a serving loop, graph capture): one
 * tiny launch on `stream` moves the sticky device flags into *dst (device memory, or pinned
 * host memory from hipHostMalloc) and clears them; the host reads *dst once the stream has
 * passed that point.  No reference counterpart (the reference panics, src/router.rs:41). */
moe_status moe_device_flags_async(moe_ctx *ctx, uint32_t *dst, void *stream);

/* Poll rounds after which a bounded wait inside moe_decode_stack expires (default 65536;
 * a round is one reload of the awaited words).  0 makes every wait that is not satisfied at
 * its first look expire at once -- a host-forced timeout for testing the failure path, in
 * which every workgroup still exits normally.  No reference counterpart. */
moe_status moe_stack_spin_limit(moe_ctx *ctx, uint32_t polls);

/* Per-phase timeline of moe_decode_stack (profiling hook; no reference counterpart).  In a
 * library built with MOE_STACK_TRACE (libmoe680m_trace.so) every later moe_decode_stack
 * launch of this context stores, per workgroup, layer and event, the 100 MHz device clock
 * into buf (device memory, `words` u64: hidden/8 workgroups x n_layers x 16 events; the event
 * numbering is k_stack.hip's StackTraceEvent).  buf = NULL stops it.  Other builds return
 * MOE_EUNSUPPORTED. */
moe_status moe_stack_trace(moe_ctx *ctx, uint64_t *buf, size_t words);

/* Last error message of the calling thread ("" when none). */
const char *moe_last_error(void);

/* ---- per-kernel timing (profiling hook) ----
 * No reference counterpart: the reference has no timing code at all (its only figure,
 * README.md:27, is unmeasured).  While enabled with `capacity` > 0 event pairs, every
 * kernel the context launches outside stream capture is bracketed by two HIP events on
 * its own stream.  moe_timing_read waits for them, returns per kernel id the number of
 * timed launches and their summed milliseconds, and starts a new window.  Events are
 * created here, never inside a hot call; capacity 0 disables and frees them. */
enum {
    MOE_K_ROUTER_TOPK = 0,     /* moe_router_topk; moe_ffn_route's first prefill launch (routing + bucket counts) */
    MOE_K_BUCKET_FILL = 1,     /* moe_bucket_fill; the prefill chain's count launch (moe_ffn, ids given) and its
                                  placement + prep launch */
    MOE_K_DECODE_GATE_UP = 2,  /* moe_ffn / moe_ffn_route, M <= 8 */
    MOE_K_DECODE_DOWN = 3,
    MOE_K_PREFILL_GATE_UP = 4,
    MOE_K_PREFILL_DOWN = 5,
    MOE_K_PREFILL_COMBINE = 6,
    MOE_K_DECODE_STACK = 7,    /* moe_decode_stack: its one persistent launch (routing included) */
    MOE_K_ROUTER_GEMV = 8,     /* moe_router_gemv_topk: the GEMV launch (its top-8 is ROUTER_TOPK) */
    MOE_K_DECODE_PREP = 9,     /* moe_ffn / moe_ffn_route, 5 <= M <= 8: routing, plan, int8 activations */
    MOE_K_COUNT = 10
};
moe_status moe_timing_enable(moe_ctx *ctx, int capacity);
moe_status moe_timing_read(moe_ctx *ctx, int counts[MOE_K_COUNT], double total_ms[MOE_K_COUNT]);

/* ---- seeded input generators (benchmark/test utilities, not part of the drop-in) ----
 * Counter-based streams: element i of stream `seed` depends only on (seed, i). */
/* IQ4_XS super-blocks first..first+n-1: uniform nibbles, uniform 6-bit scales,
 * d = f16(|N(0,1)| * 2e-3). */
moe_status moe_gen_iq4xs(void *dst, size_t n_superblocks, uint64_t seed, uint64_t first,
                         void *stream);
/* dst[i] = mean + std * N(0,1)_(first+i). */
moe_status moe_gen_normal(float *dst, size_t n, uint64_t seed, uint64_t first, float mean,
                          float std, void *stream);
/* Router logits [M][E]: N(0,1) plus kind 0 none | 1 Zipf(param) bias over a seeded
 * expert permutation | 2 with probability param a token's hot-expert logit = hot_value. */
moe_status moe_gen_logits(float *dst, int M, int E, uint64_t seed, int kind, double param,
                          double hot_value, void *stream);

#ifdef __cplusplus
}
#endif
#endif
