// k_route.hip -- router softmax + top-8 and the prefix-sum expert bucket fill.
#include "moe_internal.hpp"
#include "bucket_fill.hpp"

namespace moe {

// ---------------------------------------------------------------- router top-8
// One 64-lane wave per token.  Replaces shaders/router_topk.comp, whose 256-lane workgroup
// ran two 8-step LDS tree reductions and a serial insertion sort on lane 0
// (router_topk.comp:37-85).  Here each lane keeps E/64 logits in registers; each of the 8
// rounds is one wave max of the order-preserving key (six DPP steps into lane 63) and a
// ballot of the lanes holding it; the lowest index holding it wins, like the shader's strict
// '>' insertion (router_topk.comp:76).  Lane r then stores rank r and its weight, lane 8 the
// shared slot.  E <= 256 (moe_create's limit), so four logits per lane.
__global__ __launch_bounds__(64) void k_router_topk(const float *__restrict__ logits, int M, int E, int renorm,
                                                    uint16_t *__restrict__ ids, float *__restrict__ w) {
    // one wave per workgroup: the dispatcher spreads the tokens over every CU and SIMD
    const int lane = threadIdx.x & 63;
    const int t = blockIdx.x;
    if (t >= M) return; // whole wave leaves together
    int id;
    float wt;
    route_wave<4>(logits + (size_t)t * E, E, renorm, lane, id, wt);
    if (lane < SLOTS) {
        ids[(size_t)t * SLOTS + lane] = (uint16_t)id;
        w[(size_t)t * SLOTS + lane] = wt;
    }
}

// The same with four waves per token (route_wg4, the same results): about 2.5 times less
// latency per token, for small M where latency, not throughput, is what a launch costs.
__global__ __launch_bounds__(256) void k_router_topk_wg4(const float *__restrict__ logits, int M, int E, int renorm,
                                                         uint16_t *__restrict__ ids, float *__restrict__ w) {
    __shared__ RouteLds R;
    const int lane = threadIdx.x & 63, wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int t = blockIdx.x;
    int id;
    float wt;
    route_wg4(logits + (size_t)t * E, E, renorm, lane, wv, R, id, wt);
    if (wv == 0 && lane < SLOTS) {
        ids[(size_t)t * SLOTS + lane] = (uint16_t)id;
        w[(size_t)t * SLOTS + lane] = wt;
    }
}

constexpr int ROUTER_WG4_MAX_M = 256;

hipError_t launch_router_topk(const float *logits, int M, int E, int renorm, uint16_t *ids, float *w,
                              hipStream_t st, KernelTimer *T) {
    if (M <= 0) return hipSuccess;
    if (E < TOPK || E > 256) return hipErrorInvalidValue;
    {
        TimedLaunch tl(T, MOE_K_ROUTER_TOPK, st);
        if (M <= ROUTER_WG4_MAX_M)
            hipLaunchKernelGGL(k_router_topk_wg4, dim3((unsigned)M), dim3(256), 0, st, logits, M, E, renorm, ids, w);
        else
            hipLaunchKernelGGL(k_router_topk, dim3((unsigned)M), dim3(64), 0, st, logits, M, E, renorm, ids, w);
    }
    return hipGetLastError();
}

// ---------------------------------------------------------------- router gate GEMV
// logits[t][e] = sum_k xin[t][k] * Wg[e][k], xin = x or RMSNorm(x); Wg [E][H], rows = experts,
// in the caller's buffer as GGML IQ4_XS (136-byte super-blocks), f32 or f16 (the types a GGUF
// file's ffn_gate_inp comes in: llama.cpp's quantizer keeps that tensor F32 or F16).
// Replaces shaders/router.comp:21-61 (dispatched at src/inference.rs:598-605), whose 64x8 f32
// tiles re-dequantized every weight per tile.  One wave per (expert row, group of TM tokens:
// 1, 2 or 4 by M), four waves per workgroup: lane l owns the 32 weights 32l..32l+31 of the
// row (H = 2048 is one sub-block per lane) and reads them once -- IQ4_XS: decoded into
// biased codebook bytes and one f32 scale; f32: eight 16-byte loads; f16: four, converted
// exactly -- then for each token takes one f32 dot of 32 against x (loaded for all the
// group's tokens before any is used) and a wave sum.  All f32: the weights are exact, so the
// logits differ from an f64 sum by f32 rounding only.
//
// The top-8 follows as a k_router_topk launch.  Measured on MI355X, one launch for both at
// M <= 8 -- the last workgroup of a token group routing it after the others' logits were
// handed over through a device counter -- was slower than two launches in a graph: 8.8 us
// at M = 1 with an agent-scope release / acquire pair (each writes back / invalidates the XCD's
// whole L2), 6.2 us with write-through stores and system-scope loads instead, against 5.6 us.
constexpr int RG_WAVES = 4; // experts per workgroup

struct RouterGemvArgs {
    const void *wg;
    const float *x;
    int M, E, rmsnorm;
    float *logits;
};

// The lane's 32 weights of row e as f32 (dense types), or its codebook bytes and scale (IQ4_XS).
template <int H, int WT>
__device__ __forceinline__ void router_row_weights(const void *wg, int e, int sl, bool on, uint32_t (&kv)[8],
                                                   float &dl, float (&wf)[32]) {
    if constexpr (WT == MOE_WG_IQ4_XS) {
        constexpr int SBR = H / QK;
        const uint8_t *blk = (const uint8_t *)wg + ((size_t)e * SBR + sl / 8) * SB_BYTES;
        const u32x2 hdr = ldg<u32x2>(blk);
        const int j = sl % 8;
        const u32x2 q01 = ldg<u32x2>(blk + 8 + 16 * j), q23 = ldg<u32x2>(blk + 16 + 16 * j);
        const uint32_t q[4] = {q01.x, q01.y, q23.x, q23.y};
#pragma unroll
        for (int d = 0; d < 4; ++d) kv_biased8(q[d], kv[2 * d], kv[2 * d + 1]);
        dl = on ? sub_scale(hdr, j) : 0.0f;
    } else if constexpr (WT == MOE_WG_F32) {
        load32((const float *)wg + (size_t)e * H + 32 * sl, wf);
        if (!on)
#pragma unroll
            for (int k = 0; k < 32; ++k) wf[k] = 0.0f;
    } else {
        const _Float16 *src = (const _Float16 *)wg + (size_t)e * H + 32 * sl;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const u32x4 v = ldg<u32x4>(src + 8 * i);
#pragma unroll
            for (int d = 0; d < 4; ++d) {
                const f16x2 h2 = __builtin_bit_cast(f16x2, (uint32_t)v[d]);
                wf[8 * i + 2 * d] = on ? (float)h2[0] : 0.0f;
                wf[8 * i + 2 * d + 1] = on ? (float)h2[1] : 0.0f;
            }
        }
    }
}

template <int H, int RG_TM, int WT>
__global__ __launch_bounds__(64 * RG_WAVES) void k_router_gemv(RouterGemvArgs a) {
    constexpr int NSB = H / 32;
    static_assert(H % QK == 0 && NSB <= 64, "one sub-block per lane");
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int e = blockIdx.x * RG_WAVES + wv;
    const int t0 = blockIdx.y * RG_TM;
    const int M = a.M, E = a.E;
    if (e < E) { // whole wave
        const bool on = lane < NSB;
        const int sl = on ? lane : 0; // idle lanes (H < 2048) read sub-block 0 and add nothing
        uint32_t kv[8];
        float dl = 0.0f, wf[32];
        router_row_weights<H, WT>(a.wg, e, sl, on, kv, dl, wf);
        float xv[RG_TM][32];
#pragma unroll
        for (int i = 0; i < RG_TM; ++i) {
            const int t = t0 + i < M ? t0 + i : M - 1; // rows past M repeat the last; not stored
            load32(a.x + (size_t)t * H + 32 * sl, xv[i]);
        }
#pragma unroll
        for (int i = 0; i < RG_TM; ++i) {
            float xs = 0.f, ss = 0.f;
#pragma unroll
            for (int k = 0; k < 32; ++k) {
                xs += xv[i][k];
                ss = __builtin_fmaf(xv[i][k], xv[i][k], ss);
            }
            float part;
            if constexpr (WT == MOE_WG_IQ4_XS) {
                part = dl * subblock_dot(kv, xv[i], xs);
            } else {
                part = 0.0f;
#pragma unroll
                for (int k = 0; k < 32; ++k) part = __builtin_fmaf(wf[k], xv[i][k], part);
            }
            const float dot = wave_sum(part);
            float inv = 1.0f;
            if (a.rmsnorm) inv = 1.0f / sqrtf(wave_sum(on ? ss : 0.0f) * (1.0f / (float)H) + 1e-6f);
            if (lane == 0 && t0 + i < M) a.logits[(size_t)(t0 + i) * E + e] = dot * inv;
        }
    }
}

template <int H, int TM, int WT>
static void launch_router_gemv_t(const RouterGemvArgs &a, hipStream_t st) {
    const dim3 grid((unsigned)((a.E + RG_WAVES - 1) / RG_WAVES), (unsigned)((a.M + TM - 1) / TM));
    hipLaunchKernelGGL((k_router_gemv<H, TM, WT>), grid, dim3(64 * RG_WAVES), 0, st, a);
}

template <int H, int WT>
static void launch_router_gemv_w(const RouterGemvArgs &a, hipStream_t st) {
    // a wave's tokens past M repeat the last one: at small M fewer tokens per wave
    if (a.M == 1) launch_router_gemv_t<H, 1, WT>(a, st);
    else if (a.M == 2) launch_router_gemv_t<H, 2, WT>(a, st);
    else launch_router_gemv_t<H, 4, WT>(a, st);
}

template <int H>
static void launch_router_gemv_h(int wtype, const RouterGemvArgs &a, hipStream_t st) {
    if (wtype == MOE_WG_IQ4_XS) launch_router_gemv_w<H, MOE_WG_IQ4_XS>(a, st);
    else if (wtype == MOE_WG_F32) launch_router_gemv_w<H, MOE_WG_F32>(a, st);
    else launch_router_gemv_w<H, MOE_WG_F16>(a, st);
}

hipError_t launch_router_gemv(int H, int wtype, const void *wg, const float *x, int M, int E, int rmsnorm,
                              float *logits, int renorm, uint16_t *ids, float *w, hipStream_t st, KernelTimer *T) {
    if (M <= 0) return hipSuccess;
    if (H != 2048 && H != 512) return hipErrorInvalidValue;
    if (wtype != MOE_WG_IQ4_XS && wtype != MOE_WG_F32 && wtype != MOE_WG_F16) return hipErrorInvalidValue;
    if (E < TOPK || E > 256) return hipErrorInvalidValue;
    RouterGemvArgs a{wg, x, M, E, rmsnorm, logits};
    {
        TimedLaunch tl(T, MOE_K_ROUTER_GEMV, st);
        if (H == 2048) launch_router_gemv_h<2048>(wtype, a, st);
        else launch_router_gemv_h<512>(wtype, a, st);
    }
    hipError_t he = hipGetLastError();
    if (he == hipSuccess && ids) he = launch_router_topk(logits, M, E, renorm, ids, w, st, T);
    return he;
}

// ---------------------------------------------------------------- bucket fill
__global__ __launch_bounds__(BF_THREADS) void k_bucket_fill(BucketArgs a) { bucket_fill_one_wg(a); }
__global__ __launch_bounds__(BF_CHUNK_THREADS) void k_bucket_count(BucketArgs a) { bucket_count_chunk(a, blockIdx.x); }
__global__ __launch_bounds__(BF_THREADS) void k_bucket_scan(BucketArgs a) { bucket_scan_wg(a); }
__global__ __launch_bounds__(BF_CHUNK_THREADS) void k_bucket_scatter(BucketArgs a) { bucket_scatter_chunk(a, blockIdx.x); }

hipError_t launch_bucket_fill(const BucketArgs &a, hipStream_t st, KernelTimer *T) {
    if (a.M < 0) return hipSuccess; // M == 0 still writes all-zero ranges
    TimedLaunch tl(T, MOE_K_BUCKET_FILL, st);
    if (bucket_one_wg(a.M, a.E1)) {
        hipLaunchKernelGGL(k_bucket_fill, dim3(1), dim3(BF_THREADS), bucket_smem_one(a.E1, a.M), st, a);
    } else {
        const dim3 grid((unsigned)((a.M + 63) / 64));
        const size_t smem = bucket_chunk_smem(a.E1);
        hipLaunchKernelGGL(k_bucket_count, grid, dim3(BF_CHUNK_THREADS), smem, st, a);
        hipLaunchKernelGGL(k_bucket_scan, dim3(1), dim3(BF_THREADS), bucket_smem(a.E1, false), st, a);
        hipLaunchKernelGGL(k_bucket_scatter, grid, dim3(BF_CHUNK_THREADS), smem, st, a);
    }
    return hipGetLastError();
}

} // namespace moe
