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
    std::vector<LayerPtrs> layers;
    std::vector<char> bound;
    void *arena = nullptr; // one device allocation, carved below
    size_t arena_bytes = 0;
    uint32_t *flags = nullptr;
    float *hbuf = nullptr;       // decode h: [8][9][I] f32
    __bf16 *xb = nullptr;        // [m_max][H]
    __bf16 *hs = nullptr;        // [9 m_max][I]
    float *part = nullptr;       // [9 m_max][H]
    uint32_t *ranges = nullptr;  // [E+2]
    uint16_t *stok = nullptr;    // [9 m_max]
    float *sw = nullptr;         // [9 m_max]
    uint32_t *pos = nullptr;     // [m_max][9]
    uint32_t *chunk = nullptr;   // [ceil(m_max/64)][E+1]
    Tile *tiles = nullptr;       // [tile_max(m_max)]
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

} // namespace

extern "C" {

const char *moe_last_error(void) { return g_err.c_str(); }

moe_status moe_create(int device, const moe_config *cfg, moe_ctx **out) {
    if (!cfg || !out) return fail(MOE_EINVAL, "moe_create: null argument");
    *out = nullptr;
    const int H = cfg->hidden, I = cfg->inter, E = cfg->n_experts;
    if (!shape_compiled(H, I))
        return fail(MOE_EUNSUPPORTED, "moe_create: hidden=%d inter=%d not compiled (2048x512, 512x256)", H, I);
    if (E < MOE_TOPK || E > 1024) return fail(MOE_EINVAL, "moe_create: n_experts=%d outside 8..1024", E);
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
    c->layers.resize(cfg->n_layers);
    c->bound.assign(cfg->n_layers, 0);

    const size_t mm = (size_t)cfg->m_max, E1 = (size_t)E + 1;
    const size_t nchunk = (mm + 63) / 64;
    const size_t tmax = (size_t)tile_max_for((int)mm, (int)E1);
    struct Part {
        void **dst;
        size_t bytes;
    } parts[] = {
        {(void **)&c->flags, 256},
        {(void **)&c->hbuf, (size_t)MOE_DECODE_MAX_M * SLOTS * I * sizeof(float)},
        {(void **)&c->xb, mm * H * 2},
        {(void **)&c->hs, SLOTS * mm * I * 2},
        {(void **)&c->part, SLOTS * mm * H * sizeof(float)},
        {(void **)&c->ranges, (E1 + 1) * 4},
        {(void **)&c->stok, SLOTS * mm * 2},
        {(void **)&c->sw, SLOTS * mm * 4},
        {(void **)&c->pos, mm * SLOTS * 4},
        {(void **)&c->chunk, nchunk * E1 * 4},
        {(void **)&c->tiles, tmax * sizeof(Tile)},
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
    he = hipMemset(c->flags, 0, 256);
    if (he == hipSuccess) he = hipDeviceSynchronize();
    if (he != hipSuccess) {
        (void)hipFree(c->arena);
        delete c;
        return hip_fail(he, "moe_create: clearing workspace");
    }
    *out = c;
    return ok();
}

moe_status moe_destroy(moe_ctx *ctx) {
    if (!ctx) return fail(MOE_EINVAL, "moe_destroy: null context");
    (void)hipSetDevice(ctx->device);
    (void)hipDeviceSynchronize();
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
    ctx->layers[layer] = L;
    ctx->bound[layer] = 1;
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
                                       w, as_stream(stream));
    if (he != hipSuccess) return hip_fail(he, "moe_router_topk: launch");
    return ok();
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
    a.tile_bm = PF_BM;
    a.flags = ctx->flags;
    hipError_t he = launch_bucket_fill(a, as_stream(stream));
    if (he != hipSuccess) return hip_fail(he, "moe_bucket_fill: launch");
    return ok();
}

moe_status moe_ffn(moe_ctx *ctx, int layer, const float *x, const uint16_t *ids, const float *w, int M,
                   float *y, int flags, void *stream) {
    if (!ctx) return fail(MOE_EINVAL, "moe_ffn: null context");
    if (layer < 0 || layer >= ctx->cfg.n_layers)
        return fail(MOE_EINVAL, "moe_ffn: layer %d outside 0..%d", layer, ctx->cfg.n_layers - 1);
    if (!ctx->bound[layer]) return fail(MOE_EINVAL, "moe_ffn: layer %d has no bound weights", layer);
    if (M < 0 || M > ctx->cfg.m_max) return fail(MOE_EINVAL, "moe_ffn: M=%d outside 0..m_max=%d", M, ctx->cfg.m_max);
    if (flags & ~(MOE_FFN_ACCUMULATE | MOE_FFN_RMSNORM)) return fail(MOE_EINVAL, "moe_ffn: unknown flags 0x%x", flags);
    if (M == 0) return ok();
    if (!x || !ids || !w || !y) return fail(MOE_EINVAL, "moe_ffn: null argument");
    if (!aligned16(x) || !aligned16(y)) return fail(MOE_EINVAL, "moe_ffn: x and y must be 16-byte aligned");
    if (((uintptr_t)w & 3u) || ((uintptr_t)ids & 1u)) return fail(MOE_EINVAL, "moe_ffn: misaligned routing");
    const int H = ctx->cfg.hidden, I = ctx->cfg.inter, E = ctx->cfg.n_experts;
    const float c = ctx->cfg.wmode == MOE_W_REF ? 1.0f / 9.0f : 1.0f;
    hipStream_t st = as_stream(stream);
    hipError_t he;
    if (M <= MOE_DECODE_MAX_M) {
        DecodeArgs a{};
        a.L = ctx->layers[layer];
        a.x = x;
        a.ids = ids;
        a.w = w;
        a.y = y;
        a.hbuf = ctx->hbuf;
        a.flags = ctx->flags;
        a.M = M;
        a.E = E;
        a.accumulate = (flags & MOE_FFN_ACCUMULATE) ? 1 : 0;
        a.rmsnorm = (flags & MOE_FFN_RMSNORM) ? 1 : 0;
        a.c = c;
        he = launch_decode(H, I, a, st);
        if (he != hipSuccess) return hip_fail(he, "moe_ffn: decode launch");
        return ok();
    }
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
    b.tile_bm = PF_BM;
    b.flags = ctx->flags;
    he = launch_bucket_fill(b, st);
    if (he != hipSuccess) return hip_fail(he, "moe_ffn: bucket fill launch");
    PrefillArgs p{};
    p.L = ctx->layers[layer];
    p.x = x;
    p.xb = ctx->xb;
    p.sorted_tok = ctx->stok;
    p.sorted_w = ctx->sw;
    p.pos = ctx->pos;
    p.tiles = ctx->tiles;
    p.hs = ctx->hs;
    p.part = ctx->part;
    p.y = y;
    p.M = M;
    p.E = E;
    p.accumulate = (flags & MOE_FFN_ACCUMULATE) ? 1 : 0;
    p.rmsnorm = (flags & MOE_FFN_RMSNORM) ? 1 : 0;
    p.tile_max = b.tile_max;
    p.c = c;
    he = launch_prefill(H, I, p, st);
    if (he != hipSuccess) return hip_fail(he, "moe_ffn: prefill launch");
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

moe_status moe_device_flags(moe_ctx *ctx, void *stream, uint32_t *flags) {
    if (!ctx || !flags) return fail(MOE_EINVAL, "moe_device_flags: null argument");
    hipError_t he = hipStreamSynchronize(as_stream(stream));
    if (he != hipSuccess) return hip_fail(he, "moe_device_flags: hipStreamSynchronize");
    uint32_t v = 0;
    he = hipMemcpy(&v, ctx->flags, 4, hipMemcpyDeviceToHost);
    if (he != hipSuccess) return hip_fail(he, "moe_device_flags: hipMemcpy");
    he = hipMemset(ctx->flags, 0, 4);
    if (he == hipSuccess) he = hipDeviceSynchronize();
    if (he != hipSuccess) return hip_fail(he, "moe_device_flags: clearing");
    *flags = v;
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
