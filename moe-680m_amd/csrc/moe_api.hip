// moe_api.hip -- the extern "C" boundary: context, validation, stream-ordered dispatch.
//
// Stands in for the MoE slice of InferenceEngine (src/inference.rs:622-766): where the
// reference records Vulkan dispatches with 128-byte push constants into one UMA arena and
// blocks on a fence per layer, this library takes device pointers and a HIP stream,
// validates on the host, launches, and returns without synchronising.  All workspaces are
// allocated once by moe_create for m_max tokens.
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <new>
#include <string>
#include <vector>

#include "moe_internal.hpp"

using namespace moe;


struct moe_ctx {
    int device = 0;
    moe_config cfg{};
    std::vector<LayerPtrs> slayers; // the library's split copy of each bound layer (every kernel)
    std::vector<char> bound;
    uint8_t *spk = nullptr;         // [n_layers][E+1][W1|W3|W2] split layout: the one resident copy
    void *arena = nullptr; // one device allocation, carved below
    size_t arena_bytes = 0;
    uint32_t *flags = nullptr;   // [0] sticky device flags, [1] the decode stack's abort word
    float *hbuf = nullptr;       // decode path h scratch [72][I]
    _Float16 *xh = nullptr;      // [m_max][H]
    float *xinv = nullptr;       // [m_max]
    _Float16 *hh = nullptr;      // [9 m_max][I]
    float *hmax = nullptr;       // [9 m_max][I/PF_NGU]
    _Float16 *part = nullptr;    // [9 m_max][H]
    int8_t *pexp = nullptr;      // [9 m_max][H/32]
    float *logits = nullptr;     // [m_max][E] router GEMV output when the caller gives none
    uint32_t *ranges = nullptr;  // [E+2]
    uint16_t *stok = nullptr;    // [9 m_max]
    float *sw = nullptr;         // [9 m_max]
    uint32_t *pos = nullptr;     // [m_max][9]
    uint32_t *chunk = nullptr;   // [ceil(m_max/64)][E+1]
    uint32_t *pcnt = nullptr;    // [PF_CNT_COPIES][E+1] the prefill chain's bucket counters (zero between calls)
    uint32_t *pslot = nullptr;   // [9 m_max] the prefill chain's slot bucket and rank
    Tile *tiles = nullptr;       // [tile_max(m_max)]
    LayerPtrs *dlayers = nullptr; // device layer table of the split copies (decode stack)
    StackRouter *drouters = nullptr;   // device table of the bound router matrices
    std::vector<StackRouter> hrouters; // ... and its host copy
    uint32_t *xtag = nullptr;    // decode stack: control words, then its two exchange sets
    size_t xtag_words = 0;
    int stack_ok = 0;            // all stack workgroups fit on the device at once
    int stack_ok_ar = 0;         // ... and those of its activation-routed form
    int ncu = 0;                 // compute units of the device
    uint32_t spin_max = STK_SPIN_DEFAULT; // decode stack: poll rounds before a wait expires
    uint64_t *trace = nullptr;   // decode stack timeline buffer (MOE_STACK_TRACE builds)
    size_t trace_words = 0;
    KernelTimer timer;
};

namespace {

thread_local std::string g_err;

moe_status fail(moe_status st, const char *fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_err = buf;
    return st;
}

moe_status ok() {
    g_err.clear();
    return MOE_OK;
}

moe_status hip_fail(hipError_t e, const char *what) {
    return fail(MOE_EHIP, "%s: %s", what, hipGetErrorString(e));
}

bool aligned16(const void *p) { return ((uintptr_t)p & 15u) == 0; }

bool shape_compiled(int H, int I) { return (H == 2048 && I == 512) || (H == 512 && I == 256); }

size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

hipStream_t as_stream(void *s) { return reinterpret_cast<hipStream_t>(s); }

// The context's timer when timing is on and the stream is not being captured into a graph
// (an event recorded during capture would become a graph dependency, not a timestamp).
KernelTimer *timer_for(moe_ctx *ctx, hipStream_t st) {
    if (ctx->timer.cap <= 0) return nullptr;
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(st, &cs) != hipSuccess || cs != hipStreamCaptureStatusNone) return nullptr;
    return &ctx->timer;
}

void timer_free(KernelTimer &T) {
    for (int i = 0; i < 2 * T.cap; ++i) (void)hipEventDestroy(T.ev[i]);
    delete[] T.ev;
    delete[] T.kid;
    T = KernelTimer{};
}

} // namespace

extern "C" {

const char *moe_last_error(void) { return g_err.c_str(); }

moe_status moe_create(int device, const moe_config *cfg, moe_ctx **out) {
    if (!cfg || !out) return fail(MOE_EINVAL, "moe_create: null argument");
    *out = nullptr;
    const int H = cfg->hidden, I = cfg->inter, E = cfg->n_experts;
    if (!shape_compiled(H, I))
        return fail(MOE_EUNSUPPORTED, "moe_create: hidden=%d inter=%d not compiled (2048x512, 512x256)", H, I);
    if (E < MOE_TOPK || E > MOE_MAX_EXPERTS)
        return fail(MOE_EINVAL, "moe_create: n_experts=%d outside %d..%d", E, MOE_TOPK, MOE_MAX_EXPERTS);
    if (cfg->n_layers < 1 || cfg->n_layers > 4096)
        return fail(MOE_EINVAL, "moe_create: n_layers=%d outside 1..4096", cfg->n_layers);
    if (cfg->m_max < 1 || cfg->m_max > 65535)
        return fail(MOE_EINVAL, "moe_create: m_max=%d outside 1..65535", cfg->m_max);
    if (cfg->wmode != MOE_W_REF && cfg->wmode != MOE_W_RENORM)
        return fail(MOE_EINVAL, "moe_create: unknown wmode %d", (int)cfg->wmode);
    int ndev = 0;
    hipError_t he = hipGetDeviceCount(&ndev);
    if (he != hipSuccess) return hip_fail(he, "moe_create: hipGetDeviceCount");
    if (device < 0 || device >= ndev) return fail(MOE_EINVAL, "moe_create: device %d of %d", device, ndev);
    if ((he = hipSetDevice(device)) != hipSuccess) return hip_fail(he, "moe_create: hipSetDevice");

    moe_ctx *c = new (std::nothrow) moe_ctx();
    if (!c) return fail(MOE_ENOMEM, "moe_create: host allocation");
    c->device = device;
    c->cfg = *cfg;
    c->slayers.resize(cfg->n_layers);
    c->bound.assign(cfg->n_layers, 0);
    c->hrouters.assign(cfg->n_layers, StackRouter{nullptr, 0u, 0u});

    const size_t mm = (size_t)cfg->m_max, E1 = (size_t)E + 1;
    const size_t nchunk = (mm + 63) / 64;
    const size_t tmax = (size_t)tile_max_for((int)mm, (int)E1);
    struct Part {
        void **dst;
        size_t bytes;
    } parts[] = {
        {(void **)&c->flags, 256},
        {(void **)&c->hbuf, decode_scratch_floats(H, I) * sizeof(float)},
        {(void **)&c->xh, mm * H * 2},
        {(void **)&c->xinv, mm * 4},
        {(void **)&c->hh, SLOTS * mm * I * 2},
        {(void **)&c->hmax, SLOTS * mm * (I / PF_NGU) * 4},
        {(void **)&c->part, SLOTS * mm * H * 2},
        {(void **)&c->pexp, SLOTS * mm * (H / 32)},
        {(void **)&c->logits, mm * (size_t)E * 4},
        {(void **)&c->ranges, (E1 + 1) * 4},
        {(void **)&c->stok, SLOTS * mm * 2},
        {(void **)&c->sw, SLOTS * mm * 4},
        {(void **)&c->pos, mm * SLOTS * 4},
        {(void **)&c->chunk, nchunk * E1 * 4},
        {(void **)&c->pcnt, (size_t)PF_CNT_COPIES * E1 * 4},
        {(void **)&c->pslot, SLOTS * mm * 4},
        {(void **)&c->tiles, tmax * sizeof(Tile)},
        {(void **)&c->dlayers, (size_t)cfg->n_layers * sizeof(LayerPtrs)},
        {(void **)&c->drouters, (size_t)cfg->n_layers * sizeof(StackRouter)},
        {(void **)&c->xtag, (STK_CTL_WORDS + 2 * (size_t)cfg->n_layers * stack_layer_words(H, I)) * 4},
    };
    size_t total = 0;
    for (auto &p : parts) total += align_up(p.bytes, 256);
    he = hipMalloc(&c->arena, total);
    if (he != hipSuccess) {
        delete c;
        return fail(MOE_ENOMEM, "moe_create: hipMalloc(%zu): %s", total, hipGetErrorString(he));
    }
    c->arena_bytes = total;
    size_t off = 0;
    for (auto &p : parts) {
        *p.dst = (char *)c->arena + off;
        off += align_up(p.bytes, 256);
    }
    {
        // every kernel family reads the library's own split copy of each bound layer
        // (k_repack_split); the caller's buffers are not read after moe_bind_layer returns
        const size_t mat = (size_t)H * I / QK * SB_BYTES;
        const size_t sbytes = (size_t)cfg->n_layers * E1 * 3 * mat;
        he = hipMalloc((void **)&c->spk, sbytes);
        if (he != hipSuccess) {
            (void)hipFree(c->arena);
            delete c;
            return fail(MOE_ENOMEM, "moe_create: hipMalloc(%zu) for the weight copies: %s", sbytes,
                        hipGetErrorString(he));
        }
    }
    c->xtag_words = STK_CTL_WORDS + 2 * (size_t)cfg->n_layers * stack_layer_words(H, I);
    he = hipMemset(c->flags, 0, 256);
    if (he == hipSuccess) he = hipMemset(c->dlayers, 0, (size_t)cfg->n_layers * sizeof(LayerPtrs));
    if (he == hipSuccess) he = hipMemset(c->drouters, 0, (size_t)cfg->n_layers * sizeof(StackRouter));
    if (he == hipSuccess) he = hipMemset(c->pcnt, 0, (size_t)PF_CNT_COPIES * E1 * 4);
    // the decode stack's control words and both exchange sets start zeroed
    if (he == hipSuccess) he = hipMemset(c->xtag, 0, c->xtag_words * 4);
    if (he == hipSuccess) he = hipDeviceSynchronize();
    if (he != hipSuccess) {
        if (c->spk) (void)hipFree(c->spk);
        (void)hipFree(c->arena);
        delete c;
        return hip_fail(he, "moe_create: clearing workspace");
    }
    // The decode stack needs every one of its workgroups resident at once.
    int per_cu = 0, ncu = 0;
    if (hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess || ncu < 1)
        ncu = 1;
    c->ncu = ncu;
    if (stack_occupancy(H, I, false, &per_cu) == hipSuccess)
        c->stack_ok = (per_cu >= 1 && (long)per_cu * ncu >= stack_blocks(H) && E <= 256) ? 1 : 0;
    per_cu = 0;
    if (stack_occupancy(H, I, true, &per_cu) == hipSuccess)
        c->stack_ok_ar = (per_cu >= 1 && (long)per_cu * ncu >= stack_blocks(H) && E <= 256) ? 1 : 0;
    // moe_ffn_noalloc's static scratch: its device address looked up now, with the device
    // current, so that entry point never makes the lookup itself (a failure here is not
    // fatal: that entry point retries and reports it)
    (void)noalloc_prepare(device);
    *out = c;
    return ok();
}

moe_status moe_destroy(moe_ctx *ctx) {
    if (!ctx) return fail(MOE_EINVAL, "moe_destroy: null context");
    (void)hipSetDevice(ctx->device);
    (void)hipDeviceSynchronize();
    timer_free(ctx->timer);
    if (ctx->spk) (void)hipFree(ctx->spk);
    hipError_t he = hipFree(ctx->arena);
    delete ctx;
    if (he != hipSuccess) return hip_fail(he, "moe_destroy: hipFree");
    return ok();
}

moe_status moe_bind_layer(moe_ctx *ctx, int layer, const moe_layer_weights *lw) {
    if (!ctx || !lw) return fail(MOE_EINVAL, "moe_bind_layer: null argument");
    if (layer < 0 || layer >= ctx->cfg.n_layers)
        return fail(MOE_EINVAL, "moe_bind_layer: layer %d outside 0..%d", layer, ctx->cfg.n_layers - 1);
    const void *ptrs[6] = {lw->w1, lw->w3, lw->w2, lw->shared_w1, lw->shared_w3, lw->shared_w2};
    for (const void *p : ptrs) {
        if (!p) return fail(MOE_EINVAL, "moe_bind_layer: null weight pointer");
        if (!aligned16(p)) return fail(MOE_EINVAL, "moe_bind_layer: weight pointer %p not 16-byte aligned", p);
    }
    if ((lw->w1_stride | lw->w3_stride | lw->w2_stride) & 15u)
        return fail(MOE_EINVAL, "moe_bind_layer: expert strides must be multiples of 16 bytes");
    const size_t mat = (size_t)ctx->cfg.hidden * ctx->cfg.inter / QK * SB_BYTES;
    if (lw->w1_stride < mat || lw->w3_stride < mat || lw->w2_stride < mat)
        return fail(MOE_EINVAL, "moe_bind_layer: expert stride below one matrix (%zu bytes)", mat);
    LayerPtrs L;
    L.w1 = (const uint8_t *)lw->w1;
    L.w3 = (const uint8_t *)lw->w3;
    L.w2 = (const uint8_t *)lw->w2;
    L.s1 = lw->w1_stride;
    L.s3 = lw->w3_stride;
    L.s2 = lw->w2_stride;
    L.sw1 = (const uint8_t *)lw->shared_w1;
    L.sw3 = (const uint8_t *)lw->shared_w3;
    L.sw2 = (const uint8_t *)lw->shared_w2;
    const int H = ctx->cfg.hidden, I = ctx->cfg.inter, E = ctx->cfg.n_experts;
    hipError_t he;
    {
        const size_t es = 3 * mat;
        uint8_t *base = ctx->spk + (size_t)layer * (E + 1) * es;
        he = launch_repack_split(L.w1, L.s1, L.sw1, base, es, E, I, H, nullptr);
        if (he == hipSuccess) he = launch_repack_split(L.w3, L.s3, L.sw3, base + mat, es, E, I, H, nullptr);
        if (he == hipSuccess) he = launch_repack_split(L.w2, L.s2, L.sw2, base + 2 * mat, es, E, H, I, nullptr);
        if (he == hipSuccess) he = hipDeviceSynchronize();
        if (he != hipSuccess) return hip_fail(he, "moe_bind_layer: repacking into the split layout");
        LayerPtrs S;
        S.w1 = base;
        S.w3 = base + mat;
        S.w2 = base + 2 * mat;
        S.s1 = S.s3 = S.s2 = es;
        S.sw1 = base + (size_t)E * es;
        S.sw3 = S.sw1 + mat;
        S.sw2 = S.sw1 + 2 * mat;
        he = hipMemcpy(ctx->dlayers + layer, &S, sizeof(LayerPtrs), hipMemcpyHostToDevice);
        if (he != hipSuccess) return hip_fail(he, "moe_bind_layer: copying the layer table");
        ctx->slayers[layer] = S;
    }
    ctx->bound[layer] = 1;
    return ok();
}

moe_status moe_bind_router(moe_ctx *ctx, int layer, const void *wg, int wg_type) {
    if (!ctx) return fail(MOE_EINVAL, "moe_bind_router: null context");
    if (layer < 0 || layer >= ctx->cfg.n_layers)
        return fail(MOE_EINVAL, "moe_bind_router: layer %d outside 0..%d", layer, ctx->cfg.n_layers - 1);
    StackRouter R{nullptr, 0u, 0u};
    if (wg) {
        if (wg_type != MOE_WG_IQ4_XS && wg_type != MOE_WG_F32 && wg_type != MOE_WG_F16)
            return fail(MOE_EUNSUPPORTED, "moe_bind_router: gate matrix type %d (IQ4_XS %d, F32 %d and F16 %d)",
                        wg_type, MOE_WG_IQ4_XS, MOE_WG_F32, MOE_WG_F16);
        if (!aligned16(wg)) return fail(MOE_EINVAL, "moe_bind_router: gate matrix %p not 16-byte aligned", wg);
        R.wg = (const uint8_t *)wg;
        R.type = (uint32_t)wg_type;
    }
    hipError_t he = hipSetDevice(ctx->device);
    if (he == hipSuccess) he = hipMemcpy(ctx->drouters + layer, &R, sizeof R, hipMemcpyHostToDevice);
    if (he != hipSuccess) return hip_fail(he, "moe_bind_router: copying the router table");
    ctx->hrouters[layer] = R;
    return ok();
}

moe_status moe_router_topk(moe_ctx *ctx, const float *logits, int M, uint16_t *ids, float *w,
                           void *stream) {
    if (!ctx) return fail(MOE_EINVAL, "moe_router_topk: null context");
    if (M < 0 || M > 65535) return fail(MOE_EINVAL, "moe_router_topk: M=%d outside 0..65535", M);
    if (M == 0) return ok();
    if (!logits || !ids || !w) return fail(MOE_EINVAL, "moe_router_topk: null argument");
    if (((uintptr_t)logits & 3u) || ((uintptr_t)w & 3u) || ((uintptr_t)ids & 1u))
        return fail(MOE_EINVAL, "moe_router_topk: misaligned pointer");
    hipError_t he = launch_router_topk(logits, M, ctx->cfg.n_experts, ctx->cfg.wmode == MOE_W_RENORM, ids,
                                       w, as_stream(stream), timer_for(ctx, as_stream(stream)));
    if (he != hipSuccess) return hip_fail(he, "moe_router_topk: launch");
    return ok();
}

moe_status moe_router_gemv_topk_typed(moe_ctx *ctx, const void *wg, int wg_type, const float *x, int M, int flags,
                                      float *logits, uint16_t *ids, float *w, void *stream) {
    static const char *fn = "moe_router_gemv_topk";
    if (!ctx) return fail(MOE_EINVAL, "%s: null context", fn);
    if (wg_type != MOE_WG_IQ4_XS && wg_type != MOE_WG_F32 && wg_type != MOE_WG_F16)
        return fail(MOE_EUNSUPPORTED, "%s: gate matrix type %d (IQ4_XS %d, F32 %d and F16 %d are read)", fn, wg_type,
                    MOE_WG_IQ4_XS, MOE_WG_F32, MOE_WG_F16);
    if (M < 0 || M > 65535) return fail(MOE_EINVAL, "%s: M=%d outside 0..65535", fn, M);
    if (flags & ~MOE_FFN_RMSNORM) return fail(MOE_EINVAL, "%s: flags 0x%x (only MOE_FFN_RMSNORM)", fn, flags);
    if (!ids != !w) return fail(MOE_EINVAL, "%s: ids and w must both be given or both be NULL", fn);
    if (!logits && !ids) return fail(MOE_EINVAL, "%s: no output (logits, ids and w all NULL)", fn);
    if (!logits && M > ctx->cfg.m_max)
        return fail(MOE_EINVAL, "%s: M=%d above m_max=%d with no logits buffer", fn, M, ctx->cfg.m_max);
    if (M == 0) return ok();
    if (!wg || !x) return fail(MOE_EINVAL, "%s: null argument", fn);
    if (!aligned16(wg) || !aligned16(x) || ((uintptr_t)logits & 3u) || ((uintptr_t)w & 3u) || ((uintptr_t)ids & 1u))
        return fail(MOE_EINVAL, "%s: misaligned pointer (wg and x need 16 bytes)", fn);
    const hipStream_t st = as_stream(stream);
    float *lg = logits ? logits : ctx->logits;
    hipError_t he = launch_router_gemv(ctx->cfg.hidden, wg_type, wg, x, M, ctx->cfg.n_experts,
                                       (flags & MOE_FFN_RMSNORM) ? 1 : 0, lg, ctx->cfg.wmode == MOE_W_RENORM, ids, w,
                                       st, timer_for(ctx, st));
    if (he != hipSuccess) return hip_fail(he, "moe_router_gemv_topk: launch");
    return ok();
}

moe_status moe_router_gemv_topk(moe_ctx *ctx, const void *wg, const float *x, int M, int flags, float *logits,
                                uint16_t *ids, float *w, void *stream) {
    return moe_router_gemv_topk_typed(ctx, wg, MOE_WG_IQ4_XS, x, M, flags, logits, ids, w, stream);
}

moe_status moe_bucket_fill(moe_ctx *ctx, const uint16_t *ids, const float *w, int M, uint32_t *ranges,
                           uint16_t *sorted_tok, float *sorted_w, void *stream) {
    if (!ctx || !ranges) return fail(MOE_EINVAL, "moe_bucket_fill: null argument");
    if (M < 0 || M > ctx->cfg.m_max)
        return fail(MOE_EINVAL, "moe_bucket_fill: M=%d outside 0..m_max=%d", M, ctx->cfg.m_max);
    if (M > 0 && (!ids || !w || !sorted_tok || !sorted_w))
        return fail(MOE_EINVAL, "moe_bucket_fill: null argument");
    BucketArgs a{};
    a.ids = ids;
    a.w = w;
    a.M = M;
    a.E1 = ctx->cfg.n_experts + 1;
    a.ranges = ranges;
    a.sorted_tok = sorted_tok;
    a.sorted_w = sorted_w;
    a.pos = nullptr;
    a.chunk_cnt = ctx->chunk;
    a.tiles = nullptr;
    a.tile_max = 0;
    a.flags = ctx->flags;
    hipError_t he = launch_bucket_fill(a, as_stream(stream), timer_for(ctx, as_stream(stream)));
    if (he != hipSuccess) return hip_fail(he, "moe_bucket_fill: launch");
    return ok();
}

// The checks and launches shared by moe_ffn and moe_ffn_route.  logits == NULL: ids/w are
// inputs; otherwise the tokens are routed first and ids/w receive the routing.  scr is the
// decode path's scratch (decode_scratch_floats(hidden, inter): h, then the plan block).
static moe_status ffn_call(const char *fn, moe_ctx *ctx, int layer, const float *x, const float *logits,
                           uint16_t *ids, float *w, int M, float *y, int flags, void *stream, float *hbuf) {
    if (!ctx) return fail(MOE_EINVAL, "%s: null context", fn);
    if (layer < 0 || layer >= ctx->cfg.n_layers)
        return fail(MOE_EINVAL, "%s: layer %d outside 0..%d", fn, layer, ctx->cfg.n_layers - 1);
    if (!ctx->bound[layer]) return fail(MOE_EINVAL, "%s: layer %d has no bound weights", fn, layer);
    if (M < 0 || M > ctx->cfg.m_max) return fail(MOE_EINVAL, "%s: M=%d outside 0..m_max=%d", fn, M, ctx->cfg.m_max);
    if (flags & ~(MOE_FFN_ACCUMULATE | MOE_FFN_RMSNORM)) return fail(MOE_EINVAL, "%s: unknown flags 0x%x", fn, flags);
    if (M == 0) return ok();
    if (!x || !ids || !w || !y) return fail(MOE_EINVAL, "%s: null argument", fn);
    if (!aligned16(x) || !aligned16(y)) return fail(MOE_EINVAL, "%s: x and y must be 16-byte aligned", fn);
    if (((uintptr_t)w & 3u) || ((uintptr_t)ids & 1u) || ((uintptr_t)logits & 3u))
        return fail(MOE_EINVAL, "%s: misaligned routing", fn);
    const int H = ctx->cfg.hidden, I = ctx->cfg.inter, E = ctx->cfg.n_experts;
    const int renorm = ctx->cfg.wmode == MOE_W_RENORM;
    const float c = renorm ? 1.0f : 1.0f / 9.0f;
    hipStream_t st = as_stream(stream);
    KernelTimer *T = timer_for(ctx, st);
    hipError_t he;
    if (M <= MOE_DECODE_MAX_M) {
        // the decode launches route the tokens themselves (M <= 4: every gate/up workgroup;
        // M >= 5: the prep launch) and publish ids/w
        DecodeArgs a{};
        a.L = ctx->slayers[layer];
        a.x = x;
        a.logits = logits;
        a.ids = ids;
        a.w = w;
        a.y = y;
        a.hbuf = hbuf;
        a.plan = hbuf + decode_hbuf_floats((size_t)I);
        a.flags = ctx->flags;
        a.M = M;
        a.E = E;
        a.accumulate = (flags & MOE_FFN_ACCUMULATE) ? 1 : 0;
        a.rmsnorm = (flags & MOE_FFN_RMSNORM) ? 1 : 0;
        a.renorm = renorm;
        a.c = c;
        // gate/up: one workgroup per CU for M = 1 (every SIMD one wave), two for M <= 4, three
        // beyond (measured best at each M)
        a.nwg = ctx->ncu * (M == 1 ? 1 : M <= 4 ? 2 : 3);
        he = launch_decode(H, I, a, st, T);
        if (he != hipSuccess) return fail(MOE_EHIP, "%s: decode launch: %s", fn, hipGetErrorString(he));
        return ok();
    }
    // with logits the chain's first launch routes the tokens (into ids / w) as it counts them
    PfCountArgs pc{};
    pc.logits = logits;
    pc.ids = ids;
    pc.w = w;
    pc.M = M;
    pc.E = E;
    pc.renorm = renorm;
    pc.cnt = ctx->pcnt;
    pc.slot = ctx->pslot;
    pc.flags = ctx->flags;
    BucketArgs b{};
    b.ids = ids;
    b.w = w;
    b.M = M;
    b.E1 = E + 1;
    b.ranges = ctx->ranges;
    b.sorted_tok = ctx->stok;
    b.sorted_w = ctx->sw;
    b.pos = ctx->pos;
    b.chunk_cnt = ctx->chunk;
    b.tiles = ctx->tiles;
    b.tile_max = tile_max_for(M, E + 1);
    b.flags = ctx->flags;
    PrefillArgs p{};
    p.L = ctx->slayers[layer];
    p.x = x;
    p.xh = ctx->xh;
    p.xinv = ctx->xinv;
    p.sorted_tok = ctx->stok;
    p.sorted_w = ctx->sw;
    p.pos = ctx->pos;
    p.tiles = ctx->tiles;
    p.hh = ctx->hh;
    p.hmax = ctx->hmax;
    p.part = ctx->part;
    p.pexp = ctx->pexp;
    p.y = y;
    p.M = M;
    p.E = E;
    p.accumulate = (flags & MOE_FFN_ACCUMULATE) ? 1 : 0;
    p.rmsnorm = (flags & MOE_FFN_RMSNORM) ? 1 : 0;
    p.tile_max = b.tile_max;
    p.c = c;
    p.cnt = ctx->pcnt;
    he = launch_prefill(H, I, b, pc, p, st, T);
    if (he != hipSuccess) return fail(MOE_EHIP, "%s: prefill launch: %s", fn, hipGetErrorString(he));
    return ok();
}

} // extern "C"

namespace moe {
moe_status ffn_with_scratch(const char *fn, moe_ctx *ctx, int layer, const float *x, const uint16_t *ids,
                            const float *w, int M, float *y, int flags, void *stream, float *hbuf) {
    return ffn_call(fn, ctx, layer, x, nullptr, const_cast<uint16_t *>(ids), const_cast<float *>(w), M, y, flags,
                    stream, hbuf);
}
int ctx_device(const moe_ctx *ctx) { return ctx->device; }
int ctx_inter(const moe_ctx *ctx) { return ctx->cfg.inter; }
moe_status set_error(moe_status st, const char *msg) { return fail(st, "%s", msg); }
} // namespace moe

extern "C" {

moe_status moe_ffn(moe_ctx *ctx, int layer, const float *x, const uint16_t *ids, const float *w, int M,
                   float *y, int flags, void *stream) {
    return ffn_call("moe_ffn", ctx, layer, x, nullptr, const_cast<uint16_t *>(ids), const_cast<float *>(w), M, y,
                    flags, stream, ctx ? ctx->hbuf : nullptr);
}

moe_status moe_ffn_route(moe_ctx *ctx, int layer, const float *x, const float *logits, int M, float *y,
                         uint16_t *ids, float *w, int flags, void *stream) {
    if (M > 0 && !logits) return fail(MOE_EINVAL, "moe_ffn_route: null logits");
    return ffn_call("moe_ffn_route", ctx, layer, x, logits, ids, w, M, y, flags, stream, ctx ? ctx->hbuf : nullptr);
}

moe_status moe_decode_stack(moe_ctx *ctx, int layer0, int n_layers, const float *x, const float *logits,
                            float *y, uint16_t *ids, float *w, int flags, void *stream) {
    if (!ctx) return fail(MOE_EINVAL, "moe_decode_stack: null context");
    const bool ar = (flags & MOE_STACK_ROUTE_GEMV) != 0;
    if (!x || !y) return fail(MOE_EINVAL, "moe_decode_stack: null argument");
    if (ar && logits) return fail(MOE_EINVAL, "moe_decode_stack: MOE_STACK_ROUTE_GEMV takes no logits");
    if (!ar && !logits) return fail(MOE_EINVAL, "moe_decode_stack: null logits (without MOE_STACK_ROUTE_GEMV)");
    if ((ids == nullptr) != (w == nullptr)) return fail(MOE_EINVAL, "moe_decode_stack: ids and w go together");
    if (n_layers < 1 || layer0 < 0 || layer0 + n_layers > ctx->cfg.n_layers)
        return fail(MOE_EINVAL, "moe_decode_stack: layers %d..%d outside 0..%d", layer0, layer0 + n_layers - 1,
                    ctx->cfg.n_layers - 1);
    for (int l = layer0; l < layer0 + n_layers; ++l)
        if (!ctx->bound[l]) return fail(MOE_EINVAL, "moe_decode_stack: layer %d has no bound weights", l);
    if (flags & ~(MOE_FFN_RMSNORM | MOE_STACK_ROUTE_GEMV))
        return fail(MOE_EINVAL, "moe_decode_stack: unknown flags 0x%x", flags);
    if (ar) {
        for (int l = layer0; l < layer0 + n_layers; ++l)
            if (!ctx->hrouters[l].wg)
                return fail(MOE_EINVAL, "moe_decode_stack: layer %d has no bound router (moe_bind_router)", l);
        if (!ctx->stack_ok_ar)
            return fail(MOE_EUNSUPPORTED, "moe_decode_stack: the activation-routed form needs %d co-resident "
                        "workgroups", stack_blocks(ctx->cfg.hidden));
    }
    if (!aligned16(x) || !aligned16(y) || ((uintptr_t)logits & 3u) || ((uintptr_t)ids & 1u) || ((uintptr_t)w & 3u))
        return fail(MOE_EINVAL, "moe_decode_stack: misaligned pointer (x, y need 16 bytes)");
    if (!ctx->stack_ok)
        return fail(MOE_EUNSUPPORTED, "moe_decode_stack: needs n_experts <= 256 and %d co-resident workgroups",
                    stack_blocks(ctx->cfg.hidden));
    const int H = ctx->cfg.hidden, I = ctx->cfg.inter;
    StackArgs a{};
    a.layers = ctx->dlayers;
    a.routers = ctx->drouters;
    a.layer0 = layer0;
    a.n_layers = n_layers;
    a.x = x;
    a.logits = logits;
    a.y = y;
    a.ids_out = ids;
    a.w_out = w;
    a.ctl = ctx->xtag;
    a.xs = ctx->xtag + STK_CTL_WORDS;
    a.n_max = ctx->cfg.n_layers;
    a.set_words = (size_t)ctx->cfg.n_layers * stack_layer_words(H, I);
    a.flags = ctx->flags;
    a.spin_max = ctx->spin_max;
    a.E = ctx->cfg.n_experts;
    a.rmsnorm = (flags & MOE_FFN_RMSNORM) ? 1 : 0;
    a.renorm = ctx->cfg.wmode == MOE_W_RENORM;
    a.c = ctx->cfg.wmode == MOE_W_REF ? 1.0f / 9.0f : 1.0f;
    a.trace = nullptr;
    if (ctx->trace) {
        if ((size_t)stack_blocks(H) * n_layers * STK_TRACE_EV > ctx->trace_words)
            return fail(MOE_EINVAL, "moe_decode_stack: %d layers do not fit the trace buffer (%zu words)", n_layers,
                        ctx->trace_words);
        a.trace = ctx->trace;
    }
    hipStream_t st = as_stream(stream);
    hipError_t he = launch_stack(H, I, a, st, timer_for(ctx, st));
    if (he != hipSuccess) return hip_fail(he, "moe_decode_stack: launch");
    return ok();
}

moe_status moe_dequant_iq4xs(const void *blocks, size_t n_superblocks, float *out, void *stream) {
    if (n_superblocks == 0) return ok();
    if (!blocks || !out) return fail(MOE_EINVAL, "moe_dequant_iq4xs: null argument");
    if (((uintptr_t)blocks & 7u) || !aligned16(out))
        return fail(MOE_EINVAL, "moe_dequant_iq4xs: blocks must be 8-byte and out 16-byte aligned");
    hipError_t he = launch_dequant(blocks, n_superblocks, out, as_stream(stream));
    if (he != hipSuccess) return hip_fail(he, "moe_dequant_iq4xs: launch");
    return ok();
}

moe_status moe_timing_enable(moe_ctx *ctx, int capacity) {
    if (!ctx) return fail(MOE_EINVAL, "moe_timing_enable: null context");
    if (capacity < 0 || capacity > (1 << 20))
        return fail(MOE_EINVAL, "moe_timing_enable: capacity %d outside 0..2^20", capacity);
    (void)hipDeviceSynchronize();
    timer_free(ctx->timer);
    if (capacity == 0) return ok();
    KernelTimer T;
    T.ev = new (std::nothrow) hipEvent_t[2 * (size_t)capacity];
    T.kid = new (std::nothrow) int[capacity];
    if (!T.ev || !T.kid) {
        delete[] T.ev;
        delete[] T.kid;
        return fail(MOE_ENOMEM, "moe_timing_enable: host allocation");
    }
    for (int i = 0; i < 2 * capacity; ++i) {
        hipError_t he = hipEventCreate(&T.ev[i]);
        if (he != hipSuccess) {
            T.cap = i / 2;
            for (int j = 0; j < i; ++j) (void)hipEventDestroy(T.ev[j]);
            delete[] T.ev;
            delete[] T.kid;
            return hip_fail(he, "moe_timing_enable: hipEventCreate");
        }
    }
    T.cap = capacity;
    ctx->timer = T;
    return ok();
}

moe_status moe_timing_read(moe_ctx *ctx, int counts[MOE_K_COUNT], double total_ms[MOE_K_COUNT]) {
    if (!ctx || !counts || !total_ms) return fail(MOE_EINVAL, "moe_timing_read: null argument");
    for (int k = 0; k < MOE_K_COUNT; ++k) {
        counts[k] = 0;
        total_ms[k] = 0.0;
    }
    KernelTimer &T = ctx->timer;
    for (int i = 0; i < T.n; ++i) {
        hipError_t he = hipEventSynchronize(T.ev[2 * i + 1]);
        float ms = 0.f;
        if (he == hipSuccess) he = hipEventElapsedTime(&ms, T.ev[2 * i], T.ev[2 * i + 1]);
        if (he != hipSuccess) return hip_fail(he, "moe_timing_read: event");
        if (T.kid[i] >= 0 && T.kid[i] < MOE_K_COUNT) {
            counts[T.kid[i]]++;
            total_ms[T.kid[i]] += ms;
        }
    }
    const int dropped = T.dropped;
    T.n = 0;
    T.dropped = 0;
    if (dropped) return fail(MOE_EINVAL, "moe_timing_read: %d launches not timed (capacity %d)", dropped, T.cap);
    return ok();
}

moe_status moe_device_flags(moe_ctx *ctx, void *stream, uint32_t *flags) {
    if (!ctx || !flags) return fail(MOE_EINVAL, "moe_device_flags: null argument");
    hipError_t he = hipStreamSynchronize(as_stream(stream));
    if (he != hipSuccess) return hip_fail(he, "moe_device_flags: hipStreamSynchronize");
    uint32_t v = 0;
    he = hipMemcpy(&v, ctx->flags, 4, hipMemcpyDeviceToHost);
    if (he != hipSuccess) return hip_fail(he, "moe_device_flags: hipMemcpy");
    // after an expired wait the decode stack's control words and exchange sets may be in any
    // state (a launch that saw one does not advance them reliably): start them over, and
    // clear the abort word (flags[1]) with them -- the epoch restarts at 0, and the tag of an
    // aborted epoch-0 launch would match the next epoch-0 launch
    he = hipMemset(ctx->flags, 0, (v & MOE_DEVFLAG_TIMEOUT) ? 8 : 4);
    if (he == hipSuccess && (v & MOE_DEVFLAG_TIMEOUT)) he = hipMemset(ctx->xtag, 0, ctx->xtag_words * 4);
    if (he == hipSuccess) he = hipDeviceSynchronize();
    if (he != hipSuccess) return hip_fail(he, "moe_device_flags: clearing");
    *flags = v;
    return ok();
}

moe_status moe_device_flags_async(moe_ctx *ctx, uint32_t *dst, void *stream) {
    if (!ctx || !dst) return fail(MOE_EINVAL, "moe_device_flags_async: null argument");
    if ((uintptr_t)dst & 3u) return fail(MOE_EINVAL, "moe_device_flags_async: dst not 4-byte aligned");
    hipError_t he = launch_flags_take(ctx->flags, dst, ctx->xtag, ctx->xtag_words, as_stream(stream));
    if (he != hipSuccess) return hip_fail(he, "moe_device_flags_async: launch");
    return ok();
}

moe_status moe_stack_trace(moe_ctx *ctx, uint64_t *buf, size_t words) {
    if (!ctx) return fail(MOE_EINVAL, "moe_stack_trace: null context");
#ifdef MOE_STACK_TRACE
    if (buf && ((uintptr_t)buf & 7u)) return fail(MOE_EINVAL, "moe_stack_trace: buffer not 8-byte aligned");
    ctx->trace = buf;
    ctx->trace_words = buf ? words : 0;
    return ok();
#else
    (void)buf;
    (void)words;
    return fail(MOE_EUNSUPPORTED, "moe_stack_trace: this library was built without MOE_STACK_TRACE "
                                  "(libmoe680m_trace.so has it)");
#endif
}

moe_status moe_stack_spin_limit(moe_ctx *ctx, uint32_t polls) {
    if (!ctx) return fail(MOE_EINVAL, "moe_stack_spin_limit: null context");
    ctx->spin_max = polls;
    return ok();
}

moe_status moe_gen_iq4xs(void *dst, size_t n_superblocks, uint64_t seed, uint64_t first, void *stream) {
    if (!dst) return fail(MOE_EINVAL, "moe_gen_iq4xs: null destination");
    if ((uintptr_t)dst & 7u) return fail(MOE_EINVAL, "moe_gen_iq4xs: destination not 8-byte aligned");
    hipError_t he = launch_gen_iq4xs(dst, n_superblocks, seed, first, as_stream(stream));
    if (he != hipSuccess) return hip_fail(he, "moe_gen_iq4xs: launch");
    return ok();
}

moe_status moe_gen_normal(float *dst, size_t n, uint64_t seed, uint64_t first, float mean, float std,
                          void *stream) {
    if (!dst) return fail(MOE_EINVAL, "moe_gen_normal: null destination");
    hipError_t he = launch_gen_normal(dst, n, seed, first, mean, std, as_stream(stream));
    if (he != hipSuccess) return hip_fail(he, "moe_gen_normal: launch");
    return ok();
}

moe_status moe_gen_logits(float *dst, int M, int E, uint64_t seed, int kind, double param, double hot_value,
                          void *stream) {
    if (!dst) return fail(MOE_EINVAL, "moe_gen_logits: null destination");
    if (M < 0 || E < 1 || E > 1024) return fail(MOE_EINVAL, "moe_gen_logits: M=%d E=%d", M, E);
    if (kind < 0 || kind > 2) return fail(MOE_EINVAL, "moe_gen_logits: unknown kind %d", kind);
    hipError_t he = launch_gen_logits(dst, M, E, seed, kind, param, hot_value, as_stream(stream));
    if (he != hipSuccess) return hip_fail(he, "moe_gen_logits: launch");
    return ok();
}

} // extern "C"
