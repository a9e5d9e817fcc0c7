// moe_noalloc.hip -- moe_ffn_noalloc: the decode path of moe_ffn (M <= MOE_DECODE_MAX_M)
// with its h scratch in a static device array instead of the context's workspace, for
// callers that must not allocate device memory (no hipMalloc, hipFree or allocating library
// call happens in it -- nor in moe_ffn's hot path, but that path's scratch is memory the
// context allocated).  No counterpart in the reference.
//
// `scratch` holds the decode path's h values, [9 * MOE_DECODE_MAX_M][inter <= 512] f32, and
// the plan block of its 2 <= M <= 8 launches (hidden <= 2048): 191,744 bytes; each GPU the
// library runs on keeps its own copy until the process ends.  On
// the host the array's name is only a stand-in for the symbol: host code never passes it to a
// kernel or a copy, but the device address hipGetSymbolAddress returns for it, looked up once
// per device (with that device current) by moe_create on that device -- so no call of this
// entry point, the first one under graph capture included, makes the lookup -- and kept in
// scratch_dev[] (a first call on a device whose lookup failed at moe_create retries it).
// Every call on a GPU shares that GPU's array; nothing in it needs to start at zero (the
// launches of a call write every h value and plan word they read), and calls that overlap on one
// GPU -- on two streams at once -- race.
#include <cstdio>
#include <mutex>

#include "moe_internal.hpp"

using namespace moe;

namespace {

constexpr int NOALLOC_MAX_INTER = 512;
constexpr size_t NOALLOC_FLOATS = decode_hbuf_floats(NOALLOC_MAX_INTER) + decode_plan_floats(DEC_MAX_H);
constexpr size_t NOALLOC_SCRATCH_BYTES = NOALLOC_FLOATS * sizeof(float);
static __device__ __align__(256) float scratch[NOALLOC_FLOATS];
static_assert(NOALLOC_FLOATS * sizeof(float) == 191744, "the size the header and the docs state");

constexpr int SCRATCH_MAX_DEVICES = 64;
std::mutex scratch_mu;
void *scratch_dev[SCRATCH_MAX_DEVICES] = {};

// This device's address of `scratch`; the lookup runs with `device` current.
hipError_t scratch_for(int device, float **out) {
    if (device < 0 || device >= SCRATCH_MAX_DEVICES) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lock(scratch_mu);
    if (!scratch_dev[device]) {
        int cur = -1;
        hipError_t he = hipGetDevice(&cur);
        if (he == hipSuccess && cur != device) he = hipSetDevice(device);
        void *p = nullptr;
        if (he == hipSuccess) he = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (cur >= 0 && cur != device) (void)hipSetDevice(cur);
        if (he != hipSuccess) return he;
        scratch_dev[device] = p;
    }
    *out = (float *)scratch_dev[device];
    return hipSuccess;
}

} // namespace

namespace moe {
hipError_t noalloc_prepare(int device) {
    float *p = nullptr;
    return scratch_for(device, &p);
}
} // namespace moe

extern "C" moe_status moe_ffn_noalloc(moe_ctx *ctx, int layer, const float *x, const uint16_t *ids, const float *w,
                                      int M, float *y, int flags, void *stream) {
    if (!ctx) return set_error(MOE_EINVAL, "moe_ffn_noalloc: null context");
    char msg[160];
    if (M < 0 || M > MOE_DECODE_MAX_M) {
        snprintf(msg, sizeof msg, "moe_ffn_noalloc: M=%d outside 0..%d (the static scratch holds %zu bytes)", M,
                 MOE_DECODE_MAX_M, NOALLOC_SCRATCH_BYTES);
        return set_error(MOE_EINVAL, msg);
    }
    if (ctx_inter(ctx) > NOALLOC_MAX_INTER)
        return set_error(MOE_EUNSUPPORTED, "moe_ffn_noalloc: inter exceeds the static scratch");
    float *hbuf = nullptr;
    const hipError_t he = scratch_for(ctx_device(ctx), &hbuf);
    if (he != hipSuccess) {
        snprintf(msg, sizeof msg, "moe_ffn_noalloc: hipGetSymbolAddress(scratch): %s", hipGetErrorString(he));
        return set_error(MOE_EHIP, msg);
    }
    return ffn_with_scratch("moe_ffn_noalloc", ctx, layer, x, ids, w, M, y, flags, stream, hbuf);
}
